// Shared device helpers for the gfx950 group-quantised INT8 matmul kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "sq8_plan.h"

namespace sq8 {


typedef int i32x4 __attribute__((ext_vector_type(4)));  // 16 int8 weights as one dwordx4

// Output epilogue of a matmul (the values match enum sq8_epilogue in include/sq8.h).
constexpr int kEpiNone = 0;
constexpr int kEpiResidual = 1;  // y = res + x.W^T (res may alias y)
constexpr int kEpiSwiglu = 2;    // W = [w1; w3] (N = 2F rows): y[M][F] = silu(x.w1^T) * (x.w3^T)
struct Epi {
  int mode;
  const float* res;
};

// silu(g) * u, written as the SwiGLU operator computes it: (g * 1/(1 + e^-g)) * u.
__device__ __forceinline__ float silu_mul(float g, float u) {
  const float sig = 1.0f / (1.0f + expf(-g));
  return (g * sig) * u;
}

// Weight addressing of the MFMA kernels: the lane's 16 bytes of group 0 of weight row `row`
// (ix::lane_woff gives the row-major and packed layouts).
__device__ __forceinline__ const int8_t* lane_wbase(const int8_t* w, int pk, int row, int K,
                                                    int lane) {
  return w + ix::lane_woff(pk, row, K, lane);
}
// Byte distance between consecutive 64-wide groups of one lane's weights.
__device__ __forceinline__ int wgroup_step(int pk) { return ix::wgroup_step(pk); }

// Hand-off of partial results between workgroups (split-K and split-KV reductions): every thread
// that stored partials runs publish_partials() before its workgroup (or wave) takes a ticket, and
// the taker of the last ticket runs acquire_partials() before reading them. The agent-scope
// release and acquire fences order the partial stores before the ticket and the loads after it
// for the compiler and the memory system alike (each XCD has its own L2).
__device__ __forceinline__ void publish_partials() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
}
__device__ __forceinline__ void acquire_partials() {
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
}

// Opt a kernel in to `bytes` of dynamic LDS (needed above 64 KiB) once per device: `done` holds
// one bit per device id below 64 (higher ids set the attribute on every call).
inline hipError_t ensure_dynamic_lds(const void* kernel, size_t bytes,
                                     std::atomic<uint64_t>& done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = dev >= 0 && dev < 64 ? uint64_t{1} << dev : 0;
  if (bit && (done.load(std::memory_order_acquire) & bit)) return hipSuccess;
  e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                          static_cast<int>(bytes));
  if (e == hipSuccess && bit) done.fetch_or(bit, std::memory_order_release);
  return e;
}

// Launchers (host side). Each returns hipSuccess or the launch error.
hipError_t launch_gemv(const float* x, const int8_t* w, const float* s, float* y, int M, int N,
                       int K, int gs, hipStream_t st);
int cu_count();
size_t mfma_workspace_bytes(int M, int N, int K);
// y = epilogue(x.W^T) (y is [M][N/2] for SwiGLU). Only when mfma_fuses_epilogue(M, N, K); other
// shapes take launch_mfma with epi.mode == kEpiNone and then launch_epilogue.
// With na, x is na->x and the activation rows are rmsnorm(x + na->res) * na->w, formed while
// the rows are packed (x + res is written back to x); only when mfma_norm_fused(M, N, K).
struct NormArgs {
  float* x;
  const float* res;  // may be null
  const float* w;
  float eps;
};
bool mfma_norm_fused(int M, int N, int K);
// pk: the weights are packed (sq8_pack_weights); only plans for which mfma_packed_ok holds.
hipError_t launch_mfma(const float* x, const int8_t* w, const float* s, float* y, int M, int N,
                       int K, int gs, void* ws, hipStream_t st, Epi epi = Epi{kEpiNone, nullptr},
                       const NormArgs* na = nullptr, int pk = 0);
bool mfma_packed_ok(int M, int N, int K);
size_t packed_workspace_bytes(int M, int N, int K, int gs);
hipError_t launch_pack_weights(const int8_t* w, int N, int K, int8_t* wp, hipStream_t st);
bool mfma_fuses_epilogue(int M, int N, int K);
hipError_t launch_epilogue(const float* t, float* y, int M, int N, Epi epi, hipStream_t st);
bool gemv_stream_fits(int M, int K);
hipError_t launch_gemv_norm(const float* x, const float* res, float* x_out, const float* nw,
                            float eps, const int8_t* w, const float* s, float* y, int N, int K,
                            int gs, hipStream_t st);
hipError_t launch_gemv_norm_swiglu(const float* x, const float* res, float* x_out,
                                  const float* nw, float eps, const int8_t* w, const float* s,
                                  float* y, int N, int K, int gs, hipStream_t st);
hipError_t launch_gemv_swiglu(const float* ab, const int8_t* w, const float* s, float* y, int N,
                              int K, int gs, hipStream_t st);
hipError_t launch_generic(const float* x, const int8_t* w, const float* s, float* y, int M, int N,
                          int K, int gs, hipStream_t st);

// MI355X hands workgroups to its 8 XCDs round robin (workgroup b runs on XCD b % 8), and each
// XCD has its own L2. This maps the hardware workgroup id to a logical one such that the logical
// ids of each aligned group of G (query heads that read one kv head) run on one XCD at nearly the
// same time, while successive groups still go round robin over the XCDs (load stays balanced).
// A bijection when the grid is a multiple of 8 * G; identity otherwise.
__device__ __forceinline__ int xcd_grouped_id(int G) {
  const int b = blockIdx.x, n = gridDim.x;
  if (G <= 1 || n % (8 * G) != 0) return b;
  const int x = b & 7, s = b >> 3;
  return ((s / G) * 8 + x) * G + s % G;
}

// Sign-extend byte `b` (0..3) of a dword and convert to fp32; exact for int8.
__device__ __forceinline__ float byte_to_f32(uint32_t d, int b) {
  return static_cast<float>(static_cast<int32_t>(d << (24 - 8 * b)) >> 24);
}

// Sum over the 16 int8 of `q` times the 16 fp32 of x[0..3]; the per-group scale is applied by
// the caller once per 16-element chunk (all 16 lie in one group when group_size % 16 == 0).
__device__ __forceinline__ float dot16(const i32x4 q, const float4 x0, const float4 x1,
                                       const float4 x2, const float4 x3) {
  const uint32_t d0 = static_cast<uint32_t>(q.x), d1 = static_cast<uint32_t>(q.y);
  const uint32_t d2 = static_cast<uint32_t>(q.z), d3 = static_cast<uint32_t>(q.w);
  float a = x0.x * byte_to_f32(d0, 0);
  float b = x0.y * byte_to_f32(d0, 1);
  a = fmaf(x0.z, byte_to_f32(d0, 2), a);
  b = fmaf(x0.w, byte_to_f32(d0, 3), b);
  a = fmaf(x1.x, byte_to_f32(d1, 0), a);
  b = fmaf(x1.y, byte_to_f32(d1, 1), b);
  a = fmaf(x1.z, byte_to_f32(d1, 2), a);
  b = fmaf(x1.w, byte_to_f32(d1, 3), b);
  a = fmaf(x2.x, byte_to_f32(d2, 0), a);
  b = fmaf(x2.y, byte_to_f32(d2, 1), b);
  a = fmaf(x2.z, byte_to_f32(d2, 2), a);
  b = fmaf(x2.w, byte_to_f32(d2, 3), b);
  a = fmaf(x3.x, byte_to_f32(d3, 0), a);
  b = fmaf(x3.y, byte_to_f32(d3, 1), b);
  a = fmaf(x3.z, byte_to_f32(d3, 2), a);
  b = fmaf(x3.w, byte_to_f32(d3, 3), b);
  return a + b;
}

}  // namespace sq8
