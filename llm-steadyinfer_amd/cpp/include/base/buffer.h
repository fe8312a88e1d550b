// Byte buffer with an optional owning allocator. Mirrors the reference's
// src/include/base/buffer.h:6-43: external (non-owning) views when constructed from a pointer with
// use_external, otherwise memory from the allocator, released on destruction.
#ifndef SQ8_OP_BASE_BUFFER_H_
#define SQ8_OP_BASE_BUFFER_H_
#include <memory>
#include "base/alloc.h"

namespace base {

class Buffer : public NoCopyable, public std::enable_shared_from_this<Buffer> {
 public:
  Buffer() = default;
  explicit Buffer(size_t byte_size, std::shared_ptr<DeviceAllocator> allocator = nullptr,
                  void* ptr = nullptr, bool use_external = false);
  virtual ~Buffer();

  bool allocate();
  // Copies min(own, other) bytes from other, choosing the copy kind from both device types.
  void copy_from(const Buffer& buffer) const;
  void copy_from(const Buffer* buffer) const;

  void* ptr() { return ptr_; }
  const void* ptr() const { return ptr_; }
  size_t byte_size() const { return byte_size_; }
  std::shared_ptr<DeviceAllocator> allocator() const { return allocator_; }
  DeviceType device_type() const { return device_type_; }
  void set_device_type(DeviceType t) { device_type_ = t; }
  std::shared_ptr<Buffer> get_shared_from_this() { return shared_from_this(); }
  bool is_external() const { return use_external_; }

 private:
  size_t byte_size_ = 0;
  void* ptr_ = nullptr;
  bool use_external_ = false;
  DeviceType device_type_ = DeviceType::kDeviceUnknown;
  std::shared_ptr<DeviceAllocator> allocator_;
};

}  // namespace base
#endif  // SQ8_OP_BASE_BUFFER_H_
