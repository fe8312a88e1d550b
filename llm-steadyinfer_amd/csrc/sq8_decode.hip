// Single-sequence decode operators for gfx950 (declared in include/sq8_decode.h).
//
// These are latency-bound at batch 1 (each touches at most a few hundred KB), so the designs aim
// at few launches and full-wave work: one workgroup per row for the norms, one per head for
// attention, vectorised elementwise kernels. Reductions run in a fixed order (wave butterflies,
// then waves in index order), so every result is deterministic.
#include <algorithm>
#include <float.h>
#include <limits.h>
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

// Sum over a workgroup of W waves; every thread gets the total. `red` holds W floats.
template <int W = kBlockWaves>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();  // red may still be read from a previous reduction
  if ((threadIdx.x & (kWave - 1)) == 0) red[wave] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int i = 1; i < W; ++i) t += red[i];
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

// The same for dim % 4 == 0 and dim <= 4 * NPT * kBlock: each thread keeps its NPT float4 of the
// row in registers, so the row is read once and written once.
template <bool ADD, int NPT>
__global__ __launch_bounds__(kBlock) void rmsnorm_vec_kernel(float* __restrict__ x,
                                                             const float* __restrict__ res,
                                                             const float* __restrict__ w,
                                                             float* __restrict__ out, int dim,
                                                             float eps) {
  __shared__ float red[kBlockWaves];
  const int n4 = dim / 4;
  float4* xr = reinterpret_cast<float4*>(x + static_cast<size_t>(blockIdx.x) * dim);
  const float4* rr = reinterpret_cast<const float4*>(res + (ADD ? static_cast<size_t>(blockIdx.x) * dim : 0));
  const float4* w4 = reinterpret_cast<const float4*>(w);
  float4* orow = reinterpret_cast<float4*>(out + static_cast<size_t>(blockIdx.x) * dim);
  float4 v[NPT];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NPT; ++k) {
    const int i = threadIdx.x + k * kBlock;
    v[k] = i < n4 ? xr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    if (ADD && i < n4) {
      const float4 r = rr[i];
      v[k] = make_float4(v[k].x + r.x, v[k].y + r.y, v[k].z + r.z, v[k].w + r.w);
    }
    ss = fmaf(v[k].x, v[k].x, ss);
    ss = fmaf(v[k].y, v[k].y, ss);
    ss = fmaf(v[k].z, v[k].z, ss);
    ss = fmaf(v[k].w, v[k].w, ss);
  }
  const float total = block_sum(ss, red);
  const float scale = rsqrtf(total / static_cast<float>(dim) + eps);
#pragma unroll
  for (int k = 0; k < NPT; ++k) {
    const int i = threadIdx.x + k * kBlock;
    if (i < n4) {
      if (ADD) xr[i] = v[k];
      const float4 g = w4[i];
      orow[i] = make_float4(scale * v[k].x * g.x, scale * v[k].y * g.y, scale * v[k].z * g.z,
                            scale * v[k].w * g.w);
    }
  }
}

template <bool ADD>
void launch_rmsnorm(float* x, const float* res, const float* w, float* out, int rows, int dim,
                    float eps, hipStream_t st) {
  const bool vec = dim % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(out) & 15) == 0 &&
                   (!ADD || (reinterpret_cast<uintptr_t>(res) & 15) == 0);
  const int n4 = dim / 4;
  if (vec && n4 <= kBlock)
    hipLaunchKernelGGL((rmsnorm_vec_kernel<ADD, 1>), dim3(rows), dim3(kBlock), 0, st, x, res, w,
                       out, dim, eps);
  else if (vec && n4 <= 4 * kBlock)
    hipLaunchKernelGGL((rmsnorm_vec_kernel<ADD, 4>), dim3(rows), dim3(kBlock), 0, st, x, res, w,
                       out, dim, eps);
  else if (vec && n4 <= 16 * kBlock)
    hipLaunchKernelGGL((rmsnorm_vec_kernel<ADD, 16>), dim3(rows), dim3(kBlock), 0, st, x, res, w,
                       out, dim, eps);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<ADD>), dim3(rows), dim3(kBlock), 0, st, x, res, w, out,
                       dim, eps);
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

// Arguments of the fused RoPE + cache write (ROPE variant of attention_decode_kernel).
struct RopeArgs {
  int dim, kv_dim;
  const float* sin_cache;
  const float* cos_cache;
  float* kcache_w;
  float* vcache_w;
};

constexpr int kAttnBlock = 1024;
constexpr int kAttnWaves = kAttnBlock / kWave;

// Split of the positions over gridDim.y workgroups per head (flash-decoding, mha_kernel.cu:
// 178-341, here with the combine in the same launch). chunk == 0: one workgroup per head.
struct SplitArgs {
  int chunk;          // positions per workgroup
  int stride;         // floats per partial: head_size + 2 (outputs, max, sum)
  float* part;        // [head_num][gridDim.y][stride]
  unsigned* tickets;  // [head_num]: zero before the first call, left zero by every call
};
// Positions per split workgroup: 16 waves x 4 positions, one load round per wave.
constexpr int kAttnSplitChunk = kAttnWaves * 4;
constexpr int kAttnSplitMax = 16;  // workgroups per head at most
constexpr int kAttnSplitMinSeq = 512;

// One workgroup (16 waves) per query head, in a single memory round trip:
//  * wave w owns the cache positions w, w + 16, w + 32, ...; lane l holds head dims l, l + 64,
//    ... of their key and value rows. Those loads do not depend on anything computed here, so the
//    first chunk of them is issued before the query is rotated and staged;
//  * a score is the lanes' partial dot products summed across the wave; softmax runs online per
//    wave (running max m, sum l and weighted value sum), so the positions need no LDS array and
//    the only barriers are the query stage and the final combine of the 16 waves:
//        M = max_w m_w,  out[d] = sum_w acc_w[d] exp(m_w - M) / sum_w l_w exp(m_w - M).
//  * with ROPE the workgroup first rotates q and the token's k (pairs (i, i + hs/2) at table
//    column 2i), the group's leader writes k and v to cache row pos, and the token's own position
//    is scored from LDS (the cache rows read are 0 .. pos-1, written by earlier steps).
//  * with a split (sp.chunk > 0) workgroup (head, c) covers positions c*chunk .. +chunk-1 of the
//    pos + 1 live ones (workgroups past the last live chunk exit at once). Each stores its
//    un-normalised outputs, max and sum (agent-scope stores, released before the ticket),
//    takes a ticket per head, and the last of the head's live chunks merges them in chunk order
//    and resets the ticket. A single live chunk writes its output directly.
template <int HS_MAX, bool ROPE>
__global__ __launch_bounds__(kAttnBlock) void attention_decode_kernel(
    const float* __restrict__ q, const float* kcache, const float* vcache,
    const int32_t* __restrict__ pos_ptr, float* __restrict__ out, int head_num, int kv_head_num,
    int head_size, RopeArgs ra, SplitArgs sp) {
  constexpr int DPL = HS_MAX / kWave;  // head dims per lane
  // Cache positions per wave per chunk (two chunks in flight). 8 measured slower at every
  // length on MI355X (32 heads of 128: 8.1 against 6.5 us at 32 positions).
  constexpr int PCH = 4;
  constexpr int W = kAttnWaves;
  __shared__ __attribute__((aligned(16))) float s_q[HS_MAX];
  __shared__ float s_k[HS_MAX];
  __shared__ float s_v[HS_MAX];
  __shared__ float s_m[W], s_l[W];
  __shared__ float s_acc[W][HS_MAX];
  __shared__ bool s_last;
  const int head = xcd_grouped_id(head_num / kv_head_num);
  const int pos = *pos_ptr;
  const int seq = pos + 1;
  const int c = blockIdx.y;
  // Short rows are not split: the merge's extra round trip costs more than the split saves
  // below kAttnSplitMinSeq positions (MI355X, 32 heads of 128: 9.4 against 6.8 us at 64).
  const int chunk = sp.chunk > 0 && seq > kAttnSplitMinSeq ? sp.chunk : seq;
  const int nlive = (seq + chunk - 1) / chunk;
  if (c >= nlive) return;  // uniform: no positions left for this chunk
  const int p0 = c * chunk, p1 = min(seq, p0 + chunk);
  const int kv_dim = kv_head_num * head_size;
  const int group = head * kv_head_num / head_num;
  const int hoff = group * head_size;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Positions read from the cache: the chunk's, without pos when pos comes from registers.
  const int cend = min(p1, ROPE ? pos : seq);
  const int ncache = max(cend - p0, 0);
  const int nmine = wave < ncache ? (ncache - 1 - wave) / W + 1 : 0;
  const int nch = (nmine + PCH - 1) / PCH;

  // Chunk c of this wave's rows into register buffer b. Branch-free: positions past the wave's
  // last (and dims past head_size) re-read a valid element and are never used.
  float kr[2][PCH][DPL], vr[2][PCH][DPL];
  const int tmax = max(cend - 1, 0);
  auto load = [&](int b, int ci) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < PCH; ++i) {
      const int t = min(p0 + wave + (ci * PCH + i) * W, tmax);
      const float* krow = kcache + static_cast<size_t>(t) * kv_dim + hoff;
      const float* vrow = vcache + static_cast<size_t>(t) * kv_dim + hoff;
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        const int d = min(lane + j * kWave, head_size - 1);
        kr[b][i][j] = krow[d];
        vr[b][i][j] = vrow[d];
      }
    }
  };
  // Both register buffers are requested before the query is staged, so a wave with up to two
  // chunks (up to 128 unsplit positions) reads the cache in the same memory round trip as the
  // query, its rotation tables and the token's k and v.
  if (nch > 0) load(0, 0);
  if (nch > 1) load(1, 1);

  if (ROPE) {
    const int half = head_size / 2;
    const bool leader = c == 0 && head == (group * head_num + kv_head_num - 1) / kv_head_num;
    for (int i = threadIdx.x; i < half; i += kAttnBlock) {
      const float fci = ra.sin_cache[static_cast<size_t>(pos) * head_size + 2 * i];
      const float fcr = ra.cos_cache[static_cast<size_t>(pos) * head_size + 2 * i];
      const float* qh = q + head * head_size;
      const float q0 = qh[i], q1 = qh[i + half];
      s_q[i] = fcr * q0 - fci * q1;
      s_q[i + half] = fcr * q1 + fci * q0;
      const float* kh = q + ra.dim + hoff;
      const float k0 = kh[i], k1 = kh[i + half];
      const float r0 = fcr * k0 - fci * k1, r1 = fcr * k1 + fci * k0;
      s_k[i] = r0;
      s_k[i + half] = r1;
      const float* vh = q + ra.dim + ra.kv_dim + hoff;
      s_v[i] = vh[i];
      s_v[i + half] = vh[i + half];
      if (leader) {
        float* krow = ra.kcache_w + static_cast<size_t>(pos) * kv_dim + hoff;
        float* vrow = ra.vcache_w + static_cast<size_t>(pos) * kv_dim + hoff;
        krow[i] = r0;
        krow[i + half] = r1;
        vrow[i] = vh[i];
        vrow[i + half] = vh[i + half];
      }
    }
  } else {
    for (int d = threadIdx.x; d < head_size; d += kAttnBlock) s_q[d] = q[head * head_size + d];
  }
  __syncthreads();

  const float scale = 1.f / sqrtf(static_cast<float>(head_size));
  float qv[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j)
    qv[j] = lane + j * kWave < head_size ? s_q[lane + j * kWave] : 0.f;
  float m = -INFINITY, l = 0.f, acc[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) acc[j] = 0.f;
  auto consume = [&](float sc, const float (&v)[DPL]) __attribute__((always_inline)) {
    const float mn = fmaxf(m, sc);
    const float f = expf(m - mn), p = expf(sc - mn);
    l = fmaf(l, f, p);
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[j] = fmaf(acc[j], f, p * v[j]);
    m = mn;
  };
  auto consume_chunk = [&](int b, int ci) __attribute__((always_inline)) {
    float part[PCH];
#pragma unroll
    for (int i = 0; i < PCH; ++i) {
      float a = 0.f;
#pragma unroll
      for (int j = 0; j < DPL; ++j) a = fmaf(qv[j], kr[b][i][j], a);
      part[i] = a;
    }
#pragma unroll
    for (int off = 32; off >= 1; off /= 2)
#pragma unroll
      for (int i = 0; i < PCH; ++i) part[i] += __shfl_xor(part[i], off, kWave);
#pragma unroll
    for (int i = 0; i < PCH; ++i)
      if (ci * PCH + i < nmine) consume(part[i] * scale, vr[b][i]);
  };
  // Register double buffer over chunks: a buffer is refilled with the chunk two ahead as soon as
  // it has been consumed (nch is wave-uniform).
  for (int ci = 0; ci < nch; ci += 2) {
    consume_chunk(0, ci);
    if (ci + 2 < nch) load(0, ci + 2);
    if (ci + 1 >= nch) break;
    consume_chunk(1, ci + 1);
    if (ci + 3 < nch) load(1, ci + 3);
  }
  if (ROPE && pos < p1 && wave == (pos - p0) % W) {  // the token's own position, from LDS
    float a = 0.f, v[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const int d = lane + j * kWave;
      a = fmaf(qv[j], d < head_size ? s_k[d] : 0.f, a);
      v[j] = d < head_size ? s_v[d] : 0.f;
    }
#pragma unroll
    for (int off = 32; off >= 1; off /= 2) a += __shfl_xor(a, off, kWave);
    consume(a * scale, v);
  }

  if (lane == 0) {
    s_m[wave] = m;
    s_l[wave] = l;
  }
#pragma unroll
  for (int j = 0; j < DPL; ++j)
    if (lane + j * kWave < head_size) s_acc[wave][lane + j * kWave] = acc[j];
  __syncthreads();
  float mx = s_m[0];
#pragma unroll
  for (int w = 1; w < W; ++w) mx = fmaxf(mx, s_m[w]);
  if (nlive == 1) {
    for (int d = threadIdx.x; d < head_size; d += kAttnBlock) {
      float o = 0.f, lt = 0.f;
#pragma unroll
      for (int w = 0; w < W; ++w) {
        const float f = s_m[w] == -INFINITY ? 0.f : expf(s_m[w] - mx);
        o = fmaf(s_acc[w][d], f, o);
        lt = fmaf(s_l[w], f, lt);
      }
      out[head * head_size + d] = o / lt;
    }
    return;
  }
  // Split: this chunk's un-normalised outputs, max and sum.
  float* pp = sp.part + (static_cast<size_t>(head) * gridDim.y + c) * sp.stride;
  for (int d = threadIdx.x; d < head_size + 1; d += kAttnBlock) {
    float o = 0.f, lt = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float f = s_m[w] == -INFINITY ? 0.f : expf(s_m[w] - mx);
      if (d < head_size) o = fmaf(s_acc[w][d], f, o);
      lt = fmaf(s_l[w], f, lt);
    }
    if (d < head_size) {
      __hip_atomic_store(pp + d, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      __hip_atomic_store(pp + head_size, mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(pp + head_size + 1, lt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  publish_partials();
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = __hip_atomic_fetch_add(sp.tickets + head, 1u, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT) == static_cast<unsigned>(nlive - 1);
  __syncthreads();
  if (!s_last) return;
  acquire_partials();
  const float* hp = sp.part + static_cast<size_t>(head) * gridDim.y * sp.stride;
  float gm = -INFINITY;
  for (int ci = 0; ci < nlive; ++ci)
    gm = fmaxf(gm, __hip_atomic_load(hp + ci * sp.stride + head_size, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT));
  for (int d = threadIdx.x; d < head_size; d += kAttnBlock) {
    float o = 0.f, lt = 0.f;
    for (int ci = 0; ci < nlive; ++ci) {
      const float* cp = hp + ci * sp.stride;
      const float f = expf(__hip_atomic_load(cp + head_size, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT) - gm);
      o = fmaf(__hip_atomic_load(cp + d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), f, o);
      lt = fmaf(__hip_atomic_load(cp + head_size + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
                f, lt);
    }
    out[head * head_size + d] = o / lt;
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(sp.tickets + head, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// First maximum over n values in one launch. Workgroup b scans the contiguous chunk
// [b * kArgmaxChunk, ...) with independent float4 loads, reduces its (value, index) pairs in a
// fixed order and publishes its winner with agent-scope relaxed stores; the last workgroup to take
// the ticket compares the winners in chunk order and writes the index, then resets the ticket.
// Order: the larger value wins; equal values keep the smaller index (std::max_element's first
// maximum). NaN never wins; if nothing wins the result is 0.
constexpr int kArgmaxChunk = kBlock * 16;

__device__ __forceinline__ bool argmax_better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// Optional decode-step tail run by the last workgroup once the winner is known: *pos += 1 and
// the winner's embedding row is copied to x (the next step's input), so a captured step needs no
// separate advance and embedding launches.
struct Advance {
  int32_t* pos;        // null: no advance
  const float* emb;    // [vocab][dim]
  int vocab, dim;
  float* x;
};

__global__ __launch_bounds__(kBlock) void argmax_kernel(const float* __restrict__ logits, int n,
                                                        int32_t* __restrict__ out,
                                                        float* __restrict__ wval,
                                                        int* __restrict__ widx,
                                                        unsigned* __restrict__ ticket,
                                                        Advance adv) {
  __shared__ float sv[kBlockWaves];
  __shared__ int si[kBlockWaves];
  __shared__ bool last;
  __shared__ int s_tok;
  const int base = blockIdx.x * kArgmaxChunk;
  float best = -INFINITY;
  int bi = INT_MAX;
  const bool vec4 = (n % 4) == 0;
  float v[16];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int i0 = base + (threadIdx.x + j * kBlock) * 4;
    if (vec4 && i0 + 3 < n) {
      const float4 f = *reinterpret_cast<const float4*>(logits + i0);
      v[4 * j] = f.x; v[4 * j + 1] = f.y; v[4 * j + 2] = f.z; v[4 * j + 3] = f.w;
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) v[4 * j + c] = i0 + c < n ? logits[i0 + c] : -INFINITY;
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int i = base + (threadIdx.x + j * kBlock) * 4 + c;
      if (i < n && (v[4 * j + c] > best || (bi == INT_MAX && v[4 * j + c] == best))) {
        best = v[4 * j + c];
        bi = i;
      }
    }
#pragma unroll
  for (int off = 32; off >= 1; off /= 2) {
    const float ov = __shfl_xor(best, off, kWave);
    const int oi = __shfl_xor(bi, off, kWave);
    if (argmax_better(ov, oi, best, bi)) {
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
    float bv = sv[0];
    int bidx = si[0];
    for (int w = 1; w < kBlockWaves; ++w)
      if (argmax_better(sv[w], si[w], bv, bidx)) {
        bv = sv[w];
        bidx = si[w];
      }
    __hip_atomic_store(wval + blockIdx.x, bv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(widx + blockIdx.x, bidx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    publish_partials();
    last = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
           gridDim.x - 1;
    if (last) {
      acquire_partials();
      float fv = -INFINITY;
      int fi = INT_MAX;
      for (unsigned b = 0; b < gridDim.x; ++b) {
        const float cv = __hip_atomic_load(wval + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int ci = __hip_atomic_load(widx + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (argmax_better(cv, ci, fv, fi)) {
          fv = cv;
          fi = ci;
        }
      }
      s_tok = fi < n ? fi : 0;
      out[0] = s_tok;
      if (adv.pos) adv.pos[0] += 1;
      __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (!adv.pos) return;  // uniform: a kernel argument
  __syncthreads();
  if (!last) return;     // uniform: published by the barrier
  const int tok = s_tok;
  if (tok < 0 || tok >= adv.vocab) return;
  const float* row = adv.emb + static_cast<size_t>(tok) * adv.dim;
  // Up to 4 float4 per thread per pass, all loads issued before the stores (a loop of dependent
  // load-store pairs costs one memory round trip per element).
  if (adv.dim % 4 == 0 && (reinterpret_cast<uintptr_t>(row) & 15) == 0 &&
      (reinterpret_cast<uintptr_t>(adv.x) & 15) == 0) {
    const float4* r4 = reinterpret_cast<const float4*>(row);
    float4* x4 = reinterpret_cast<float4*>(adv.x);
    const int n4 = adv.dim / 4;
    for (int i0 = 0; i0 < n4; i0 += 4 * kBlock) {
      float4 v[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = i0 + j * kBlock + threadIdx.x;
        v[j] = i < n4 ? r4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = i0 + j * kBlock + threadIdx.x;
        if (i < n4) x4[i] = v[j];
      }
    }
  } else {
    for (int i = threadIdx.x; i < adv.dim; i += kBlock) adv.x[i] = row[i];
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
  launch_rmsnorm<false>(const_cast<float*>(x), nullptr, w, out, rows, dim, eps,
                        stream_of(hip_stream));
  return launched();
}

int sq8_add_rmsnorm(float* x, const float* res, const float* w, float* out, int rows, int dim,
                    float eps, void* hip_stream) {
  if (!x || !res || !w || !out) return SQ8_ERR_NULL;
  if (rows <= 0 || dim <= 0) return SQ8_ERR_DIMS;
  launch_rmsnorm<true>(x, res, w, out, rows, dim, eps, stream_of(hip_stream));
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
  if (max_seq > (1 << 24)) return SQ8_ERR_DIMS;
  if (head_size <= 128)
    hipLaunchKernelGGL((attention_decode_kernel<128, false>), dim3(head_num), dim3(kAttnBlock), 0,
                       stream_of(hip_stream), q, key_cache, value_cache, pos, out, head_num,
                       kv_head_num, head_size, RopeArgs{}, SplitArgs{});
  else
    hipLaunchKernelGGL((attention_decode_kernel<256, false>), dim3(head_num), dim3(kAttnBlock), 0,
                       stream_of(hip_stream), q, key_cache, value_cache, pos, out, head_num,
                       kv_head_num, head_size, RopeArgs{}, SplitArgs{});
  return launched();
}

int sq8_rope_attention_decode(const float* qkv, int head_num, int kv_head_num, int head_size,
                              const int32_t* pos, const float* sin_cache, const float* cos_cache,
                              float* key_cache, float* value_cache, float* out, int max_seq,
                              void* hip_stream) {
  return sq8_rope_attention_decode_ws(qkv, head_num, kv_head_num, head_size, pos, sin_cache,
                                      cos_cache, key_cache, value_cache, out, max_seq, nullptr, 0,
                                      hip_stream);
}

// Workgroups per head of the split decode attention for a cache of max_seq rows, and the
// positions each covers (a multiple of kAttnSplitChunk).
static void decode_split(int max_seq, int& chunks, int& chunk) {
  chunks = std::min((max_seq + kAttnSplitChunk - 1) / kAttnSplitChunk, kAttnSplitMax);
  const int per = (max_seq + chunks - 1) / chunks;
  chunk = (per + kAttnSplitChunk - 1) / kAttnSplitChunk * kAttnSplitChunk;
}

size_t sq8_decode_attention_workspace_bytes(int head_num, int head_size, int max_seq) {
  if (head_num <= 0 || head_size <= 0 || head_size > 256 || max_seq <= 0) return 0;
  int chunks, chunk;
  decode_split(max_seq, chunks, chunk);
  if (chunks < 2) return 0;
  const size_t tickets = (static_cast<size_t>(head_num) * 4 + 255) / 256 * 256;
  return tickets + static_cast<size_t>(head_num) * chunks * (head_size + 2) * sizeof(float);
}

int sq8_rope_attention_decode_ws(const float* qkv, int head_num, int kv_head_num, int head_size,
                                 const int32_t* pos, const float* sin_cache,
                                 const float* cos_cache, float* key_cache, float* value_cache,
                                 float* out, int max_seq, void* workspace, size_t workspace_bytes,
                                 void* hip_stream) {
  if (!qkv || !pos || !sin_cache || !cos_cache || !key_cache || !value_cache || !out)
    return SQ8_ERR_NULL;
  if (head_num <= 0 || kv_head_num <= 0 || head_num % kv_head_num || head_size <= 0 ||
      head_size % 2 || head_size > 256 || max_seq <= 0)
    return SQ8_ERR_DIMS;
  if (max_seq > (1 << 24)) return SQ8_ERR_DIMS;
  const size_t need = sq8_decode_attention_workspace_bytes(head_num, head_size, max_seq);
  if (workspace && workspace_bytes < need) return SQ8_ERR_WORKSPACE;
  const RopeArgs ra{head_num * head_size, kv_head_num * head_size, sin_cache, cos_cache, key_cache,
                    value_cache};
  SplitArgs sp{};
  int chunks = 1;
  if (workspace && need > 0) {
    int chunk;
    decode_split(max_seq, chunks, chunk);
    const size_t tickets = (static_cast<size_t>(head_num) * 4 + 255) / 256 * 256;
    sp = SplitArgs{chunk, head_size + 2,
                   reinterpret_cast<float*>(static_cast<char*>(workspace) + tickets),
                   static_cast<unsigned*>(workspace)};
  }
  const dim3 grid(head_num, chunks);
  if (head_size <= 128)
    hipLaunchKernelGGL((attention_decode_kernel<128, true>), grid, dim3(kAttnBlock), 0,
                       stream_of(hip_stream), qkv, key_cache, value_cache, pos, out, head_num,
                       kv_head_num, head_size, ra, sp);
  else
    hipLaunchKernelGGL((attention_decode_kernel<256, true>), grid, dim3(kAttnBlock), 0,
                       stream_of(hip_stream), qkv, key_cache, value_cache, pos, out, head_num,
                       kv_head_num, head_size, ra, sp);
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

size_t sq8_argmax_workspace_bytes(int n) {
  if (n <= 0) return 0;
  const size_t blocks = (static_cast<size_t>(n) + kArgmaxChunk - 1) / kArgmaxChunk;
  return 256 + blocks * (sizeof(float) + sizeof(int));
}

int sq8_argmax(const float* logits, int n, int32_t* out, void* workspace, size_t workspace_bytes,
               void* hip_stream) {
  if (!logits || !out) return SQ8_ERR_NULL;
  if (n <= 0) return SQ8_ERR_DIMS;
  if (!workspace || workspace_bytes < sq8_argmax_workspace_bytes(n)) return SQ8_ERR_WORKSPACE;
  const int blocks = (n + kArgmaxChunk - 1) / kArgmaxChunk;
  unsigned* ticket = static_cast<unsigned*>(workspace);
  float* wval = reinterpret_cast<float*>(static_cast<char*>(workspace) + 256);
  int* widx = reinterpret_cast<int*>(wval + blocks);
  hipLaunchKernelGGL(argmax_kernel, dim3(blocks), dim3(kBlock), 0, stream_of(hip_stream), logits,
                     n, out, wval, widx, ticket, Advance{});
  return launched();
}

int sq8_argmax_advance(const float* logits, int n, void* workspace, size_t workspace_bytes,
                       int32_t* pos, int32_t* token, const float* emb_table, int vocab, int dim,
                       float* x, void* hip_stream) {
  if (!logits || !pos || !token || !emb_table || !x) return SQ8_ERR_NULL;
  if (n <= 0 || vocab <= 0 || dim <= 0) return SQ8_ERR_DIMS;
  if (!workspace || workspace_bytes < sq8_argmax_workspace_bytes(n)) return SQ8_ERR_WORKSPACE;
  const int blocks = (n + kArgmaxChunk - 1) / kArgmaxChunk;
  unsigned* ticket = static_cast<unsigned*>(workspace);
  float* wval = reinterpret_cast<float*>(static_cast<char*>(workspace) + 256);
  int* widx = reinterpret_cast<int*>(wval + blocks);
  hipLaunchKernelGGL(argmax_kernel, dim3(blocks), dim3(kBlock), 0, stream_of(hip_stream), logits,
                     n, token, wval, widx, ticket, Advance{pos, emb_table, vocab, dim, x});
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
