// Allocators and copies of the op API (reference: src/source/base/alloc.cpp, alloc_cpu.cpp,
// alloc_cu.cpp). The HIP allocator caches freed blocks per device: blocks over 1 MiB are reused
// only for requests of the same rounded size class, smaller ones by best fit; a failed hipMalloc
// returns all cached blocks and retries once.
#include <hip/hip_runtime.h>
#include <cstdlib>
#include <cstring>
#include "base/alloc.h"

namespace base {

namespace {
hipMemcpyKind to_hip_kind(MemcpyKind k) {
  switch (k) {
    case MemcpyKind::kMemcpyCPU2CUDA: return hipMemcpyHostToDevice;
    case MemcpyKind::kMemcpyCUDA2CPU: return hipMemcpyDeviceToHost;
    case MemcpyKind::kMemcpyCUDA2CUDA: return hipMemcpyDeviceToDevice;
    default: return hipMemcpyHostToHost;
  }
}
constexpr size_t kBigBlock = 1u << 20;
// Sizes above kBigBlock are rounded up to 1 MiB multiples so freed blocks can serve later
// requests of a similar size.
size_t round_size(size_t b) { return b > kBigBlock ? (b + kBigBlock - 1) & ~(kBigBlock - 1) : b; }
}  // namespace

void DeviceAllocator::memcpy(const void* src_ptr, void* dest_ptr, size_t byte_size,
                             MemcpyKind memcpy_kind, void* stream, bool need_sync) const {
  CHECK_NE(src_ptr, nullptr);
  CHECK_NE(dest_ptr, nullptr);
  if (!byte_size) return;
  if (memcpy_kind == MemcpyKind::kMemcpyCPU2CPU) {
    std::memcpy(dest_ptr, src_ptr, byte_size);
    return;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = st ? hipMemcpyAsync(dest_ptr, src_ptr, byte_size, to_hip_kind(memcpy_kind), st)
                    : hipMemcpy(dest_ptr, src_ptr, byte_size, to_hip_kind(memcpy_kind));
  CHECK(e == hipSuccess) << hipGetErrorString(e);
  // Only the stream that owns the copy is synchronised, never the whole device.
  if (need_sync && st) CHECK(hipStreamSynchronize(st) == hipSuccess);
}

void DeviceAllocator::memset_zero(void* ptr, size_t byte_size, void* stream, bool need_sync) {
  CHECK(device_type_ != DeviceType::kDeviceUnknown);
  if (device_type_ == DeviceType::kDeviceCPU) {
    std::memset(ptr, 0, byte_size);
    return;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = st ? hipMemsetAsync(ptr, 0, byte_size, st) : hipMemset(ptr, 0, byte_size);
  CHECK(e == hipSuccess) << hipGetErrorString(e);
  if (need_sync && st) CHECK(hipStreamSynchronize(st) == hipSuccess);
}

void* CPUDeviceAllocator::allocate(size_t byte_size) const {
  if (!byte_size) return nullptr;
  void* p = nullptr;
  const size_t align = byte_size >= 1024 ? 64 : 16;
  if (posix_memalign(&p, align, byte_size) != 0) return nullptr;
  return p;
}

void CPUDeviceAllocator::release(void* ptr) const { std::free(ptr); }

HIPDeviceAllocator::~HIPDeviceAllocator() { free_idle(); }

void* HIPDeviceAllocator::allocate(size_t byte_size) const {
  if (byte_size == 0) return nullptr;
  int dev = 0;
  CHECK(hipGetDevice(&dev) == hipSuccess);
  const size_t want = round_size(byte_size);
  {
    std::lock_guard<std::mutex> lk(mu_);
    auto& cache = idle_[dev];
    auto it = cache.lower_bound(want);
    // Small requests take the smallest cached block that fits; big ones only their size class
    // (a huge cached block is not handed to a small request).
    if (it != cache.end() && (want <= kBigBlock ? it->first < 2 * want + kBigBlock : it->first == want)) {
      void* p = it->second;
      const size_t bytes = it->first;
      cache.erase(it);
      in_use_[p] = Block{p, bytes, dev};
      return p;
    }
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, want);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    free_idle();
    e = hipMalloc(&p, want);
  }
  if (e != hipSuccess) {
    (void)hipGetLastError();
    LOG_ERROR << "hipMalloc of " << (want >> 20) << " MiB failed: " << hipGetErrorString(e);
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(mu_);
  in_use_[p] = Block{p, want, dev};
  return p;
}

void HIPDeviceAllocator::release(void* ptr) const {
  if (!ptr) return;
  std::lock_guard<std::mutex> lk(mu_);
  auto it = in_use_.find(ptr);
  if (it == in_use_.end()) {
    LOG_WARNING << "release of a pointer this allocator does not own; freeing directly";
    CHECK(hipFree(ptr) == hipSuccess);
    return;
  }
  idle_[it->second.device].emplace(it->second.bytes, ptr);
  in_use_.erase(it);
}

void HIPDeviceAllocator::free_idle() const {
  std::lock_guard<std::mutex> lk(mu_);
  int cur = 0;
  (void)hipGetDevice(&cur);
  for (auto& kv : idle_) {
    if (kv.second.empty()) continue;
    (void)hipSetDevice(kv.first);
    for (auto& b : kv.second) (void)hipFree(b.second);
    kv.second.clear();
  }
  (void)hipSetDevice(cur);
}

size_t HIPDeviceAllocator::idle_bytes() const {
  std::lock_guard<std::mutex> lk(mu_);
  int dev = 0;
  (void)hipGetDevice(&dev);
  size_t n = 0;
  auto it = idle_.find(dev);
  if (it != idle_.end())
    for (auto& b : it->second) n += b.first;
  return n;
}

std::shared_ptr<CPUDeviceAllocator> CPUDeviceAllocatorFactory::get_instance() {
  static std::shared_ptr<CPUDeviceAllocator> inst = std::make_shared<CPUDeviceAllocator>();
  return inst;
}

std::shared_ptr<HIPDeviceAllocator> HIPDeviceAllocatorFactory::get_instance() {
  static std::shared_ptr<HIPDeviceAllocator> inst = std::make_shared<HIPDeviceAllocator>();
  return inst;
}

}  // namespace base
