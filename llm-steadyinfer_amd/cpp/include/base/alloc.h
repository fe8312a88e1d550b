// Device allocators of the op API. Mirrors the reference's src/include/base/alloc.h:14-100
// (DeviceAllocator, CPUDeviceAllocator, the device allocator and their singleton factories) with a
// HIP device allocator. HIPDeviceAllocator keeps freed blocks in per-device caches (exact-size
// reuse for blocks above 1 MiB, best fit below) so steady-state decode does no hipMalloc.
#ifndef SQ8_OP_BASE_ALLOC_H_
#define SQ8_OP_BASE_ALLOC_H_
#include <map>
#include <memory>
#include <mutex>
#include <vector>
#include "base/base.h"

namespace base {

enum class MemcpyKind {
  kMemcpyCPU2CPU = 0,
  kMemcpyCPU2CUDA = 1,
  kMemcpyCUDA2CPU = 2,
  kMemcpyCUDA2CUDA = 3,
};

class DeviceAllocator {
 public:
  explicit DeviceAllocator(DeviceType device_type) : device_type_(device_type) {}
  virtual ~DeviceAllocator() = default;
  virtual DeviceType device_type() const { return device_type_; }
  virtual void release(void* ptr) const = 0;
  virtual void* allocate(size_t byte_size) const = 0;
  // Copies byte_size bytes; with a stream the copy is asynchronous on it unless need_sync.
  virtual void memcpy(const void* src_ptr, void* dest_ptr, size_t byte_size,
                      MemcpyKind memcpy_kind = MemcpyKind::kMemcpyCPU2CPU, void* stream = nullptr,
                      bool need_sync = false) const;
  virtual void memset_zero(void* ptr, size_t byte_size, void* stream, bool need_sync = false);

 private:
  DeviceType device_type_ = DeviceType::kDeviceUnknown;
};

class CPUDeviceAllocator : public DeviceAllocator {
 public:
  CPUDeviceAllocator() : DeviceAllocator(DeviceType::kDeviceCPU) {}
  void* allocate(size_t byte_size) const override;
  void release(void* ptr) const override;
};

class HIPDeviceAllocator : public DeviceAllocator {
 public:
  HIPDeviceAllocator() : DeviceAllocator(DeviceType::kDeviceHIP) {}
  ~HIPDeviceAllocator() override;
  void* allocate(size_t byte_size) const override;
  void release(void* ptr) const override;
  // Returns every cached (not in use) block to the device.
  void free_idle() const;
  // Bytes currently held in the caches (not in use) on the current device.
  size_t idle_bytes() const;

 private:
  struct Block {
    void* ptr;
    size_t bytes;
    int device;
  };
  mutable std::mutex mu_;
  mutable std::map<void*, Block> in_use_;
  mutable std::map<int, std::multimap<size_t, void*>> idle_;  // device -> size -> block
};
using CUDADeviceAllocator = HIPDeviceAllocator;

class CPUDeviceAllocatorFactory {
 public:
  static std::shared_ptr<CPUDeviceAllocator> get_instance();
};

class HIPDeviceAllocatorFactory {
 public:
  static std::shared_ptr<HIPDeviceAllocator> get_instance();
};
using CUDADeviceAllocatorFactory = HIPDeviceAllocatorFactory;

}  // namespace base
#endif  // SQ8_OP_BASE_ALLOC_H_
