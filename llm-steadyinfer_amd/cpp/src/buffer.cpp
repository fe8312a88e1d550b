// Buffer (reference: src/source/base/buffer.cpp).
#include "base/buffer.h"

namespace base {

Buffer::Buffer(size_t byte_size, std::shared_ptr<DeviceAllocator> allocator, void* ptr,
               bool use_external)
    : byte_size_(byte_size), ptr_(ptr), use_external_(use_external), allocator_(allocator) {
  if (!ptr_ && allocator_) {
    device_type_ = allocator_->device_type();
    use_external_ = false;
    ptr_ = allocator_->allocate(byte_size);
  }
}

Buffer::~Buffer() {
  if (!use_external_ && ptr_ && allocator_) allocator_->release(ptr_);
  ptr_ = nullptr;
}

bool Buffer::allocate() {
  if (!allocator_ || byte_size_ == 0) return false;
  use_external_ = false;
  ptr_ = allocator_->allocate(byte_size_);
  return ptr_ != nullptr;
}

void Buffer::copy_from(const Buffer& other) const { copy_from(&other); }

void Buffer::copy_from(const Buffer* other) const {
  CHECK(allocator_ != nullptr);
  CHECK(other != nullptr && other->ptr_ != nullptr);
  const size_t n = byte_size_ < other->byte_size_ ? byte_size_ : other->byte_size_;
  const DeviceType src = other->device_type(), dst = device_type();
  CHECK(src != DeviceType::kDeviceUnknown && dst != DeviceType::kDeviceUnknown);
  MemcpyKind kind = MemcpyKind::kMemcpyCUDA2CUDA;
  if (src == DeviceType::kDeviceCPU && dst == DeviceType::kDeviceCPU) kind = MemcpyKind::kMemcpyCPU2CPU;
  else if (src == DeviceType::kDeviceHIP && dst == DeviceType::kDeviceCPU) kind = MemcpyKind::kMemcpyCUDA2CPU;
  else if (src == DeviceType::kDeviceCPU && dst == DeviceType::kDeviceHIP) kind = MemcpyKind::kMemcpyCPU2CUDA;
  allocator_->memcpy(other->ptr_, ptr_, n, kind);
}

}  // namespace base
