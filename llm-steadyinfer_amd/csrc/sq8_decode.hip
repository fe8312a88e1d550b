// Single-sequence decode operators for gfx950 (declared in include/sq8_decode.h).
//
// These are latency-bound at batch 1 (each touches at most a few hundred KB), so the designs aim
// at few launches and full-wave work: one workgroup per row for the norms, one per head for
// attention, vectorised elementwise kernels. Reductions run in a fixed order (wave butterflies,
// then waves in index order), so every result is deterministic.
#include <float.h>
#include <math.h>
#include "sq8.h"
#include "sq8_common.h"
#include "sq8_decode.h"

namespace sq8 {
namespace {

constexpr int kBlock = 256;
constexpr int kBlockWaves = kBlock / kWave;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off /= 2) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off /= 2) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Sum over the workgroup (kBlock threads); every thread gets the total. `red` holds kBlockWaves.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();  // red may still be read from a previous reduction
  if ((threadIdx.x & (kWave - 1)) == 0) red[wave] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int i = 1; i < kBlockWaves; ++i) t += red[i];
  return t;
}

__device__ __forceinline__ float block_max(float v, float* red) {
  v = wave_max(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & (kWave - 1)) == 0) red[wave] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int i = 1; i < kBlockWaves; ++i) t = fmaxf(t, red[i]);
  return t;
}

__global__ __launch_bounds__(kBlock) void embedding_kernel(const float* __restrict__ table,
                                                           int vocab, int dim,
                                                           const int32_t* __restrict__ tokens,
                                                           float* __restrict__ out) {
  const int i = blockIdx.x;
  const int token = tokens[i];
  if (token < 0 || token >= vocab) return;
  const float* src = table + static_cast<size_t>(token) * dim;
  float* dst = out + static_cast<size_t>(i) * dim;
  for (int d = threadIdx.x; d < dim; d += kBlock) dst[d] = src[d];
}

// ADD: x += res first (written back), then normalise x.
template <bool ADD>
__global__ __launch_bounds__(kBlock) void rmsnorm_kernel(float* __restrict__ x,
                                                         const float* __restrict__ res,
                                                         const float* __restrict__ w,
                                                         float* __restrict__ out, int dim,
                                                         float eps) {
  __shared__ float red[kBlockWaves];
  float* xr = x + static_cast<size_t>(blockIdx.x) * dim;
  float* orow = out + static_cast<size_t>(blockIdx.x) * dim;
  float ss = 0.f;
  for (int d = threadIdx.x; d < dim; d += kBlock) {
    float v = xr[d];
    if (ADD) {
      v += res[static_cast<size_t>(blockIdx.x) * dim + d];
      xr[d] = v;  // each thread re-reads only its own elements below
    }
    ss = fmaf(v, v, ss);
  }
  const float total = block_sum(ss, red);
  const float scale = rsqrtf(total / static_cast<float>(dim) + eps);
  for (int d = threadIdx.x; d < dim; d += kBlock) orow[d] = scale * xr[d] * w[d];
}

__global__ void rope_tables_kernel(float* __restrict__ sin_cache, float* __restrict__ cos_cache,
                                   int head_size, int max_seq, float theta) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= head_size * max_seq) return;
  const int pos = idx / head_size, j = idx % head_size;
  const float freq = 1.0f / powf(theta, static_cast<float>(j) / static_cast<float>(head_size));
  const float val = static_cast<float>(pos) * freq;
  sin_cache[idx] = sinf(val);
  cos_cache[idx] = cosf(val);
}

// One thread per rotation pair of q; threads whose head lies inside kv_dim also rotate the pair
// of k and copy the matching v elements into the caches.
__global__ void rope_kv_kernel(float* __restrict__ qkv, int dim, int kv_dim, int head_size,
                               const int32_t* __restrict__ pos_ptr,
                               const float* __restrict__ sin_cache,
                               const float* __restrict__ cos_cache, float* __restrict__ kcache,
                               float* __restrict__ vcache) {
  const int half = head_size / 2;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (dim / head_size) * half) return;
  const int pos = *pos_ptr;
  const int head = idx / half, i = idx % half;
  const int v0 = head * head_size + i, v1 = v0 + half;
  const float fci = sin_cache[static_cast<size_t>(pos) * head_size + 2 * i];
  const float fcr = cos_cache[static_cast<size_t>(pos) * head_size + 2 * i];
  float* q = qkv;
  const float q0 = q[v0], q1 = q[v1];
  q[v0] = fcr * q0 - fci * q1;
  q[v1] = fcr * q1 + fci * q0;
  if (head * head_size < kv_dim) {
    const float* k = qkv + dim;
    const float* v = qkv + dim + kv_dim;
    const float k0 = k[v0], k1 = k[v1];
    float* krow = kcache + static_cast<size_t>(pos) * kv_dim;
    float* vrow = vcache + static_cast<size_t>(pos) * kv_dim;
    krow[v0] = fcr * k0 - fci * k1;
    krow[v1] = fcr * k1 + fci * k0;
    vrow[v0] = v[v0];
    vrow[v1] = v[v1];
  }
}

// One workgroup per query head. Scores: wave w takes positions w, w + 4, ...; its lanes split the
// head dimension and a butterfly sums the dot product. Softmax over the scores in LDS, then
// thread d accumulates sum_t p_t * V[t][d] (coalesced across d) and divides by the sum.
template <int HS_MAX>
__global__ __launch_bounds__(kBlock) void attention_decode_kernel(
    const float* __restrict__ q, const float* __restrict__ kcache,
    const float* __restrict__ vcache, const int32_t* __restrict__ pos_ptr,
    float* __restrict__ out, int head_num, int kv_head_num, int head_size) {
  extern __shared__ float s_p[];  // [seq] scores, then probabilities
  __shared__ float red[kBlockWaves];
  __shared__ float s_q[HS_MAX];
  const int head = blockIdx.x;
  const int seq = *pos_ptr + 1;
  const int kv_dim = kv_head_num * head_size;
  const int hoff = (head * kv_head_num / head_num) * head_size;
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x >> 6;
  for (int d = threadIdx.x; d < head_size; d += kBlock) s_q[d] = q[head * head_size + d];
  __syncthreads();
  const float scale = 1.f / sqrtf(static_cast<float>(head_size));
  for (int t = wave; t < seq; t += kBlockWaves) {
    const float* krow = kcache + static_cast<size_t>(t) * kv_dim + hoff;
    float dot = 0.f;
    for (int d = lane; d < head_size; d += kWave) dot = fmaf(s_q[d], krow[d], dot);
    dot = wave_sum(dot);
    if (lane == 0) s_p[t] = dot * scale;
  }
  __syncthreads();
  float m = -FLT_MAX;
  for (int t = threadIdx.x; t < seq; t += kBlock) m = fmaxf(m, s_p[t]);
  m = block_max(m, red);
  float l = 0.f;
  for (int t = threadIdx.x; t < seq; t += kBlock) {
    const float p = expf(s_p[t] - m);
    s_p[t] = p;
    l += p;
  }
  l = block_sum(l, red);  // its barriers also publish the probabilities
  for (int d = threadIdx.x; d < head_size; d += kBlock) {
    const float* vcol = vcache + hoff + d;
    float acc = 0.f;
    for (int t = 0; t < seq; ++t) acc = fmaf(s_p[t], vcol[static_cast<size_t>(t) * kv_dim], acc);
    out[head * head_size + d] = acc / l;
  }
}

__global__ void swiglu_kernel(const float* __restrict__ a, const float* __restrict__ b,
                              float* out, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = a[i];
  const float sig = 1.0f / (1.0f + expf(-v));
  out[i] = (v * sig) * b[i];
}

__global__ void add_kernel(float* __restrict__ x, const float* __restrict__ y, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) x[i] += y[i];
}

// First maximum: each thread scans increasing indices keeping strict improvements, then the
// workgroup reduces (value, index) pairs, preferring the larger value and, on ties, the smaller
// index.
constexpr int kArgmaxBlock = 1024;
__global__ __launch_bounds__(kArgmaxBlock) void argmax_kernel(const float* __restrict__ logits,
                                                              int n, int32_t* __restrict__ out) {
  __shared__ float sv[kArgmaxBlock / kWave];
  __shared__ int si[kArgmaxBlock / kWave];
  float best = -INFINITY;
  int bi = n;  // "none yet"
  for (int i = threadIdx.x; i < n; i += kArgmaxBlock) {
    const float v = logits[i];
    if (v > best || (bi == n && v == best)) {
      best = v;
      bi = i;
    }
  }
  auto better = [](float v, int i, float bv, int bidx) {
    return v > bv || (v == bv && i < bidx);
  };
#pragma unroll
  for (int off = 32; off >= 1; off /= 2) {
    const float ov = __shfl_xor(best, off, kWave);
    const int oi = __shfl_xor(bi, off, kWave);
    if (better(ov, oi, best, bi)) {
      best = ov;
      bi = oi;
    }
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & (kWave - 1)) == 0) {
    sv[wave] = best;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = sv[0];
    int idx = si[0];
    for (int w = 1; w < kArgmaxBlock / kWave; ++w)
      if (better(sv[w], si[w], v, idx)) {
        v = sv[w];
        idx = si[w];
      }
    out[0] = idx < n ? idx : 0;
  }
}

// One thread per group: absmax, s = absmax / 127, q = round-half-away(w / s) from the fp32
// quotient (|w/s| + 0.5 is exact in fp32 for |w/s| <= 127.5).
__global__ void quantize_kernel(const float* __restrict__ w, int64_t ngroups, int gs,
                                int8_t* __restrict__ q, float* __restrict__ s) {
  const int64_t g = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (g >= ngroups) return;
  const float* wg = w + g * gs;
  float amax = 0.f;
  for (int i = 0; i < gs; ++i) amax = fmaxf(amax, fabsf(wg[i]));
  const float sc = amax / 127.0f;
  s[g] = sc;
  int8_t* qg = q + g * gs;
  for (int i = 0; i < gs; ++i) {
    if (sc == 0.f) {
      qg[i] = 0;
      continue;
    }
    const float v = wg[i] / sc;
    const float r = fminf(floorf(fabsf(v) + 0.5f), 127.0f);
    qg[i] = static_cast<int8_t>(v < 0.f ? -r : r);
  }
}

__global__ void step_advance_kernel(int32_t* pos, int32_t* token, const int32_t* next) {
  pos[0] += 1;
  token[0] = next[0];
}

int launched() { return hipGetLastError() == hipSuccess ? SQ8_OK : SQ8_ERR_LAUNCH; }
hipStream_t stream_of(void* s) { return static_cast<hipStream_t>(s); }

}  // namespace
}  // namespace sq8

using namespace sq8;

extern "C" {

int sq8_embedding(const float* table, int vocab, int dim, const int32_t* tokens, int n, float* out,
                  void* hip_stream) {
  if (!table || !tokens || !out) return SQ8_ERR_NULL;
  if (vocab <= 0 || dim <= 0 || n <= 0) return SQ8_ERR_DIMS;
  hipLaunchKernelGGL(embedding_kernel, dim3(n), dim3(kBlock), 0, stream_of(hip_stream), table,
                     vocab, dim, tokens, out);
  return launched();
}

int sq8_rmsnorm(const float* x, const float* w, float* out, int rows, int dim, float eps,
                void* hip_stream) {
  if (!x || !w || !out) return SQ8_ERR_NULL;
  if (rows <= 0 || dim <= 0) return SQ8_ERR_DIMS;
  hipLaunchKernelGGL((rmsnorm_kernel<false>), dim3(rows), dim3(kBlock), 0, stream_of(hip_stream),
                     const_cast<float*>(x), nullptr, w, out, dim, eps);
  return launched();
}

int sq8_add_rmsnorm(float* x, const float* res, const float* w, float* out, int rows, int dim,
                    float eps, void* hip_stream) {
  if (!x || !res || !w || !out) return SQ8_ERR_NULL;
  if (rows <= 0 || dim <= 0) return SQ8_ERR_DIMS;
  hipLaunchKernelGGL((rmsnorm_kernel<true>), dim3(rows), dim3(kBlock), 0, stream_of(hip_stream),
                     x, res, w, out, dim, eps);
  return launched();
}

int sq8_rope_tables(float* sin_cache, float* cos_cache, int head_size, int max_seq, float theta,
                    void* hip_stream) {
  if (!sin_cache || !cos_cache) return SQ8_ERR_NULL;
  if (head_size <= 0 || max_seq <= 0 || !(theta > 0.f)) return SQ8_ERR_DIMS;
  const int total = head_size * max_seq;
  hipLaunchKernelGGL(rope_tables_kernel, dim3((total + kBlock - 1) / kBlock), dim3(kBlock), 0,
                     stream_of(hip_stream), sin_cache, cos_cache, head_size, max_seq, theta);
  return launched();
}

int sq8_rope_kv(float* qkv, int dim, int kv_dim, int head_size, const int32_t* pos,
                const float* sin_cache, const float* cos_cache, float* key_cache,
                float* value_cache, int max_seq, void* hip_stream) {
  if (!qkv || !pos || !sin_cache || !cos_cache || !key_cache || !value_cache) return SQ8_ERR_NULL;
  if (dim <= 0 || kv_dim <= 0 || head_size <= 0 || head_size % 2 || dim % head_size ||
      kv_dim % head_size || kv_dim > dim || max_seq <= 0)
    return SQ8_ERR_DIMS;
  const int pairs = dim / 2;
  hipLaunchKernelGGL(rope_kv_kernel, dim3((pairs + kBlock - 1) / kBlock), dim3(kBlock), 0,
                     stream_of(hip_stream), qkv, dim, kv_dim, head_size, pos, sin_cache,
                     cos_cache, key_cache, value_cache);
  return launched();
}

int sq8_attention_decode(const float* q, const float* key_cache, const float* value_cache,
                         const int32_t* pos, float* out, int head_num, int kv_head_num,
                         int head_size, int max_seq, void* hip_stream) {
  if (!q || !key_cache || !value_cache || !pos || !out) return SQ8_ERR_NULL;
  if (head_num <= 0 || kv_head_num <= 0 || head_num % kv_head_num || head_size <= 0 ||
      head_size > 256 || max_seq <= 0)
    return SQ8_ERR_DIMS;
  const size_t lds = static_cast<size_t>(max_seq) * sizeof(float);
  if (lds > 64 * 1024) return SQ8_ERR_DIMS;  // scores of one head live in LDS
  hipLaunchKernelGGL((attention_decode_kernel<256>), dim3(head_num), dim3(kBlock), lds,
                     stream_of(hip_stream), q, key_cache, value_cache, pos, out, head_num,
                     kv_head_num, head_size);
  return launched();
}

int sq8_swiglu(const float* a, const float* b, float* out, int n, void* hip_stream) {
  if (!a || !b || !out) return SQ8_ERR_NULL;
  if (n <= 0) return SQ8_ERR_DIMS;
  hipLaunchKernelGGL(swiglu_kernel, dim3((n + kBlock - 1) / kBlock), dim3(kBlock), 0,
                     stream_of(hip_stream), a, b, out, n);
  return launched();
}

int sq8_add(float* x, const float* y, int n, void* hip_stream) {
  if (!x || !y) return SQ8_ERR_NULL;
  if (n <= 0) return SQ8_ERR_DIMS;
  hipLaunchKernelGGL(add_kernel, dim3((n + kBlock - 1) / kBlock), dim3(kBlock), 0,
                     stream_of(hip_stream), x, y, n);
  return launched();
}

int sq8_argmax(const float* logits, int n, int32_t* out, void* hip_stream) {
  if (!logits || !out) return SQ8_ERR_NULL;
  if (n <= 0) return SQ8_ERR_DIMS;
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(kArgmaxBlock), 0, stream_of(hip_stream), logits,
                     n, out);
  return launched();
}

int sq8_quantize(const float* w, int64_t numel, int group_size, int8_t* q, float* scales,
                 void* hip_stream) {
  if (!w || !q || !scales) return SQ8_ERR_NULL;
  if (numel <= 0) return SQ8_ERR_DIMS;
  if (group_size <= 0 || numel % group_size) return SQ8_ERR_GROUP;
  const int64_t ngroups = numel / group_size;
  const int64_t blocks = (ngroups + kBlock - 1) / kBlock;
  if (blocks > 0x7fffffff) return SQ8_ERR_DIMS;
  hipLaunchKernelGGL(quantize_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kBlock), 0,
                     stream_of(hip_stream), w, ngroups, group_size, q, scales);
  return launched();
}

int sq8_step_advance(int32_t* pos, int32_t* token, const int32_t* next, void* hip_stream) {
  if (!pos || !token || !next) return SQ8_ERR_NULL;
  hipLaunchKernelGGL(step_advance_kernel, dim3(1), dim3(1), 0, stream_of(hip_stream), pos, token,
                     next);
  return launched();
}

}  // extern "C"
