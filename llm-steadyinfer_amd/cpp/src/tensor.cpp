// Tensor (reference: src/source/tensor/tensor.cpp).
#include "tensor/tensor.h"
#include <numeric>

namespace tensor {

namespace {
size_t product(const std::vector<int32_t>& dims) {
  if (dims.empty()) return 0;
  size_t n = 1;
  for (int32_t d : dims) n *= static_cast<size_t>(d);
  return n;
}
}  // namespace

Tensor::Tensor(base::DataType data_type, int32_t dim0, bool need_alloc,
               std::shared_ptr<base::DeviceAllocator> alloc, void* ptr)
    : Tensor(data_type, std::vector<int32_t>{dim0}, need_alloc, alloc, ptr) {}

Tensor::Tensor(base::DataType data_type, int32_t dim0, int32_t dim1, bool need_alloc,
               std::shared_ptr<base::DeviceAllocator> alloc, void* ptr)
    : Tensor(data_type, std::vector<int32_t>{dim0, dim1}, need_alloc, alloc, ptr) {}

Tensor::Tensor(base::DataType data_type, int32_t dim0, int32_t dim1, int32_t dim2,
               bool need_alloc, std::shared_ptr<base::DeviceAllocator> alloc, void* ptr)
    : Tensor(data_type, std::vector<int32_t>{dim0, dim1, dim2}, need_alloc, alloc, ptr) {}

Tensor::Tensor(base::DataType data_type, std::vector<int32_t> dims, bool need_alloc,
               std::shared_ptr<base::DeviceAllocator> alloc, void* ptr)
    : size_(product(dims)), dims_(std::move(dims)), data_type_(data_type) {
  if (need_alloc && alloc) {
    allocate(alloc);
  } else if (ptr != nullptr || alloc) {
    CHECK(!(need_alloc && ptr)) << "need_alloc with an external pointer";
    init_buffer(alloc, data_type_, need_alloc, ptr);
  }
}

void Tensor::init_buffer(std::shared_ptr<base::DeviceAllocator> alloc, base::DataType data_type,
                         bool need_alloc, void* ptr) {
  if (!alloc && !need_alloc) {
    buffer_ = std::make_shared<base::Buffer>(base::DataTypeSize(data_type) * size_, nullptr, ptr,
                                             true);
  } else {
    allocate(alloc, true);
  }
}

void Tensor::to_hip(hipStream_t stream) {
  CHECK(buffer_ != nullptr);
  const base::DeviceType t = device_type();
  if (t == base::DeviceType::kDeviceUnknown) {
    LOG_ERROR << "to_hip: the tensor's device type is unknown";
  } else if (t == base::DeviceType::kDeviceCPU) {
    auto alloc = base::HIPDeviceAllocatorFactory::get_instance();
    auto dev = std::make_shared<base::Buffer>(byte_size(), alloc);
    CHECK(dev->ptr() != nullptr) << "device allocation of " << byte_size() << " bytes";
    alloc->memcpy(buffer_->ptr(), dev->ptr(), byte_size(), base::MemcpyKind::kMemcpyCPU2CUDA,
                  stream);
    buffer_ = dev;
  }
}

void Tensor::to_cpu() {
  CHECK(buffer_ != nullptr);
  const base::DeviceType t = device_type();
  if (t == base::DeviceType::kDeviceUnknown) {
    LOG_ERROR << "to_cpu: the tensor's device type is unknown";
  } else if (t == base::DeviceType::kDeviceHIP) {
    auto alloc = base::CPUDeviceAllocatorFactory::get_instance();
    auto host = std::make_shared<base::Buffer>(byte_size(), alloc);
    alloc->memcpy(buffer_->ptr(), host->ptr(), byte_size(), base::MemcpyKind::kMemcpyCUDA2CPU);
    buffer_ = host;
  }
}

bool Tensor::is_empty() const { return size_ == 0 || !buffer_ || buffer_->ptr() == nullptr; }

int32_t Tensor::get_dim(int32_t idx) const {
  CHECK_GE(idx, 0);
  CHECK_LT(idx, dims_size());
  return dims_[idx];
}

base::DeviceType Tensor::device_type() const {
  return buffer_ ? buffer_->device_type() : base::DeviceType::kDeviceUnknown;
}

void Tensor::set_device_type(base::DeviceType t) const {
  if (buffer_) buffer_->set_device_type(t);
}

bool Tensor::assign(std::shared_ptr<base::Buffer> buffer) {
  if (!buffer) {
    LOG_ERROR << "assign: null buffer";
    return false;
  }
  if (byte_size() > buffer->byte_size()) {
    LOG_ERROR << "assign: buffer of " << buffer->byte_size() << " bytes is smaller than the tensor ("
              << byte_size() << " bytes)";
    return false;
  }
  buffer_ = buffer;
  return true;
}

bool Tensor::allocate(std::shared_ptr<base::DeviceAllocator> allocator, bool need_realloc) {
  if (!allocator) {
    LOG_ERROR << "allocate: null allocator";
    return false;
  }
  if (byte_size() == 0) {
    LOG_ERROR << "allocate: the tensor has zero bytes";
    return false;
  }
  if (buffer_ && byte_size() <= buffer_->byte_size() && !need_realloc) return true;
  buffer_ = std::make_shared<base::Buffer>(byte_size(), allocator, nullptr);
  return buffer_->ptr() != nullptr;
}

void Tensor::reset(base::DataType data_type, const std::vector<int32_t>& dims) {
  data_type_ = data_type;
  dims_ = dims;
  size_ = product(dims);
  buffer_ = nullptr;
}

void Tensor::reshape(const std::vector<int32_t>& dims) {
  const size_t n = product(dims);
  if (buffer_ && n > size_) {
    auto bigger = std::make_shared<base::Buffer>(n * base::DataTypeSize(data_type_),
                                                 buffer_->allocator());
    CHECK(bigger->ptr() != nullptr);
    bigger->set_device_type(buffer_->device_type());
    bigger->copy_from(buffer_.get());
    buffer_ = bigger;
  }
  dims_ = dims;
  size_ = n;
}

std::vector<size_t> Tensor::strides() const {
  std::vector<size_t> s(dims_.size(), 1);
  for (int i = static_cast<int>(dims_.size()) - 2; i >= 0; --i) s[i] = s[i + 1] * dims_[i + 1];
  return s;
}

Tensor Tensor::clone() const {
  Tensor t = *this;
  CHECK(buffer_ && buffer_->allocator()) << "clone needs an owning buffer";
  t.buffer_ = std::make_shared<base::Buffer>(byte_size(), buffer_->allocator());
  t.buffer_->set_device_type(buffer_->device_type());
  t.buffer_->copy_from(buffer_.get());
  return t;
}

}  // namespace tensor
