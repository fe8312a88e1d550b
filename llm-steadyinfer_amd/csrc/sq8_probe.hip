// Measurement probe: a read-only streaming kernel that bounds what any kernel reading the same
// bytes once can reach on this GPU (launch, ramp-up and tail included). It has no counterpart in
// the reference; bench.py times it next to the decode GEMV at each projection's size.
#include "../../include/sq8_probe.h"
#include "../../include/sq8.h"
#include "sq8_common.h"

namespace {

using sq8::i32x4;

// Each lane reads U 16-byte chunks per iteration, all issued before any is used (nontemporal,
// as the GEMV streams its weights); the grid strides over the buffer. The words are summed as
// wrapping uint32 (order-independent) and workgroup b adds its total to sink[b % sink_len] (one
// counter for all workgroups would serialise thousands of atomics at the end), so nothing can
// be optimised away and the result is checkable.
template <int U>
__global__ __launch_bounds__(256) void stream_read_kernel(const i32x4* __restrict__ p,
                                                          size_t n16, unsigned* sink,
                                                          int sink_len) {
  const size_t stride = static_cast<size_t>(gridDim.x) * 256 * U;
  unsigned acc = 0;
  for (size_t base = static_cast<size_t>(blockIdx.x) * 256 * U + threadIdx.x; base < n16;
       base += stride) {
    i32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t i = base + static_cast<size_t>(u) * 256;
      v[u] = i < n16 ? __builtin_nontemporal_load(p + i) : i32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
      acc += static_cast<unsigned>(v[u].x) + static_cast<unsigned>(v[u].y) +
             static_cast<unsigned>(v[u].z) + static_cast<unsigned>(v[u].w);
  }
#pragma unroll
  for (int off = 32; off >= 1; off /= 2) acc += __shfl_xor(acc, off, sq8::kWave);
  __shared__ unsigned red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) atomicAdd(sink + blockIdx.x % sink_len, red[0] + red[1] + red[2] + red[3]);
}

}  // namespace

extern "C" int sq8_probe_stream_read(const void* p, size_t bytes, unsigned* sink, int sink_len,
                                     int workgroups_per_cu, int chunks_per_lane,
                                     void* hip_stream) {
  if (!p || !sink) return SQ8_ERR_NULL;
  if (sink_len <= 0) return SQ8_ERR_DIMS;
  if (bytes == 0 || bytes % 16 || (reinterpret_cast<uintptr_t>(p) & 15) ||
      workgroups_per_cu <= 0 || workgroups_per_cu > 32)
    return SQ8_ERR_DIMS;
  const size_t n16 = bytes / 16;
  const hipStream_t st = static_cast<hipStream_t>(hip_stream);
  const auto go = [&](auto kern, int U) {
    const size_t per_wg = static_cast<size_t>(256) * U;
    const size_t need = (n16 + per_wg - 1) / per_wg;
    const size_t cap = static_cast<size_t>(workgroups_per_cu) * sq8::cu_count();
    const unsigned grid = static_cast<unsigned>(need < cap ? need : cap);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256), 0, st, static_cast<const i32x4*>(p), n16,
                       sink, sink_len);
  };
  switch (chunks_per_lane) {
    case 1: go(stream_read_kernel<1>, 1); break;
    case 2: go(stream_read_kernel<2>, 2); break;
    case 4: go(stream_read_kernel<4>, 4); break;
    case 8: go(stream_read_kernel<8>, 8); break;
    default: return SQ8_ERR_DIMS;
  }
  return hipGetLastError() == hipSuccess ? SQ8_OK : SQ8_ERR_LAUNCH;
}
