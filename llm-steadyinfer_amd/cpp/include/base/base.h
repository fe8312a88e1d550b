// Core types of the op API: device/data enums, Status and error constructors, CHECK/LOG macros.
// Mirrors the reference's src/include/base/base.h:49-149 (same names and meanings) with a HIP
// device in place of CUDA; the glog dependency is replaced by the small macros below.
#ifndef SQ8_OP_BASE_BASE_H_
#define SQ8_OP_BASE_BASE_H_
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <sstream>
#include <string>

#define UNUSED(expr) \
  do {               \
    (void)(expr);    \
  } while (0)

namespace base {

// kDeviceHIP takes the value the reference gives kDeviceCUDA (base.h:49-53); kDeviceCUDA remains
// as an alias so reference call sites compile unchanged.
enum class DeviceType : uint8_t {
  kDeviceUnknown = 0,
  kDeviceCPU = 1,
  kDeviceHIP = 2,
  kDeviceCUDA = kDeviceHIP,
};

enum class DataType : uint8_t {
  kDataTypeUnknown = 0,
  kDataTypeFp32 = 1,
  kDataTypeInt8 = 2,
  kDataTypeInt32 = 3,
};

inline size_t DataTypeSize(DataType t) {
  switch (t) {
    case DataType::kDataTypeFp32: return 4;
    case DataType::kDataTypeInt8: return 1;
    case DataType::kDataTypeInt32: return 4;
    default: return 0;
  }
}

class NoCopyable {
 protected:
  NoCopyable() = default;
  ~NoCopyable() = default;
  NoCopyable(const NoCopyable&) = delete;
  NoCopyable& operator=(const NoCopyable&) = delete;
};

enum StatusCode : uint8_t {
  kSuccess = 0,
  kFunctionUnImplement = 1,
  kPathNotValid = 2,
  kModelParseError = 3,
  kInternalError = 5,
  kKeyValueHasExist = 6,
  kInvalidArgument = 7,
};

class Status {
 public:
  Status(int code = StatusCode::kSuccess, std::string err_message = "")
      : code_(code), message_(std::move(err_message)) {}
  Status& operator=(int code) {
    code_ = code;
    return *this;
  }
  bool operator==(int code) const { return code_ == code; }
  bool operator!=(int code) const { return code_ != code; }
  operator int() const { return code_; }
  operator bool() const { return code_ == kSuccess; }
  int32_t get_err_code() const { return code_; }
  const std::string& get_err_msg() const { return message_; }
  void set_err_msg(const std::string& m) { message_ = m; }

 private:
  int code_ = StatusCode::kSuccess;
  std::string message_;
};

namespace error {
inline Status Success(const std::string& m = "") { return Status(kSuccess, m); }
inline Status FunctionNotImplement(const std::string& m = "") { return Status(kFunctionUnImplement, m); }
inline Status PathNotValid(const std::string& m = "") { return Status(kPathNotValid, m); }
inline Status ModelParseError(const std::string& m = "") { return Status(kModelParseError, m); }
inline Status InternalError(const std::string& m = "") { return Status(kInternalError, m); }
inline Status KeyHasExits(const std::string& m = "") { return Status(kKeyValueHasExist, m); }
inline Status InvalidArgument(const std::string& m = "") { return Status(kInvalidArgument, m); }
}  // namespace error

namespace detail {
// Streams a fatal message and aborts when destroyed (the role glog's LOG(FATAL) plays).
class FatalStream {
 public:
  FatalStream(const char* file, int line, const char* what) {
    os_ << file << ":" << line << " " << what << " ";
  }
  [[noreturn]] ~FatalStream() {
    std::fprintf(stderr, "%s\n", os_.str().c_str());
    std::fflush(stderr);
    std::abort();
  }
  template <typename T>
  FatalStream& operator<<(const T& v) {
    os_ << v;
    return *this;
  }

 private:
  std::ostringstream os_;
};
class NullStream {
 public:
  template <typename T>
  NullStream& operator<<(const T&) {
    return *this;
  }
};
class WarnStream {
 public:
  WarnStream(const char* file, int line) { os_ << file << ":" << line << " "; }
  ~WarnStream() { std::fprintf(stderr, "%s\n", os_.str().c_str()); }
  template <typename T>
  WarnStream& operator<<(const T& v) {
    os_ << v;
    return *this;
  }

 private:
  std::ostringstream os_;
};
}  // namespace detail

#define SQ8_FATAL(what) ::base::detail::FatalStream(__FILE__, __LINE__, what)
#define CHECK(cond) \
  if (!(cond)) SQ8_FATAL("Check failed: " #cond)
#define CHECK_EQ(a, b) CHECK((a) == (b))
#define CHECK_NE(a, b) CHECK((a) != (b))
#define CHECK_GE(a, b) CHECK((a) >= (b))
#define CHECK_LT(a, b) CHECK((a) < (b))
#define LOG_FATAL SQ8_FATAL("FATAL")
#define LOG_ERROR ::base::detail::WarnStream(__FILE__, __LINE__)
#define LOG_WARNING ::base::detail::WarnStream(__FILE__, __LINE__)
#define VLOG_1 ::base::detail::NullStream()

#define STATUS_CHECK(call)                                                              \
  do {                                                                                  \
    const ::base::Status& status_ = (call);                                             \
    if (!status_) {                                                                     \
      SQ8_FATAL("Infer error") << "code " << int(status_) << ": " << status_.get_err_msg(); \
    }                                                                                   \
  } while (0)

}  // namespace base
#endif  // SQ8_OP_BASE_BASE_H_
