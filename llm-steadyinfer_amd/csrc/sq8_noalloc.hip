// sq8_matmul_noalloc: the quantised matmul for callers that cannot allocate device memory (code
// under graph capture, tight serving loops, harnesses that forbid hipMalloc). The workspace that
// sq8_matmul takes as an argument (split-K tickets, packed activations, split-K partials) lives
// here in a file-scope device array of fixed size, one copy per GPU, held until the process ends.
#include <mutex>

#include "../../include/sq8.h"
#include "sq8_common.h"

namespace {

constexpr size_t kScratchBytes = SQ8_NOALLOC_SCRATCH_BYTES;
static_assert(kScratchBytes % 256 == 0 && kScratchBytes >= sq8::kWsTicketBytes, "scratch size");

// The array's name is a host-side stand-in in host code: kernels get the per-device address
// that hipGetSymbolAddress returns, never `scratch` itself.
__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};  // per device: the address of its copy of `scratch`

// The current device's scratch address, looked up once per device. The split-K tickets at its
// start need no clearing: `scratch` has static storage, zero when the code object is loaded on a
// device, and every matmul leaves its tickets zero. So no call issues a memset or fill, and the
// first call on a device may be the one made under graph capture.
int scratch_for_current_device(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return SQ8_ERR_DEVICE;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return SQ8_ERR_DEVICE;
    g_ptr[dev] = p;
  }
  *out = g_ptr[dev];
  return SQ8_OK;
}

}  // namespace

extern "C" {

size_t sq8_noalloc_scratch_bytes(void) { return kScratchBytes; }

int sq8_matmul_noalloc(const float* x, const int8_t* w, const float* scales, float* y, int M,
                       int N, int K, int group_size, void* hip_stream) {
  if (!x || !w || !scales || !y) return SQ8_ERR_NULL;
  if (M <= 0 || N <= 0 || K <= 0 || K % 4 != 0) return SQ8_ERR_DIMS;
  if (group_size <= 0 || (static_cast<int64_t>(N) * K) % group_size != 0) return SQ8_ERR_GROUP;
  const size_t need = sq8_workspace_bytes(M, N, K, group_size);
  if (need > kScratchBytes) return SQ8_ERR_WORKSPACE;
  void* ws = nullptr;
  const int r = scratch_for_current_device(&ws);
  if (r != SQ8_OK) return r;
  return sq8_matmul(x, w, scales, y, M, N, K, group_size, ws, kScratchBytes, hip_stream);
}

}  // extern "C"
