// Continuous-batching operators (paged KV cache) for gfx950: rows of different sequences, each at
// its own position, in one launch. C ABI in include/sq8_batch.h.
#include <float.h>
#include <limits.h>
#include <math.h>

#include "sq8.h"
#include "sq8_batch.h"
#include "sq8_common.h"

namespace sq8 {
namespace {

constexpr int kBlock = 256;
constexpr int kAttnWaves = 8;  // waves per (row, head) attention workgroup

hipStream_t stream_of(void* s) { return static_cast<hipStream_t>(s); }
int launched() { return hipGetLastError() == hipSuccess ? SQ8_OK : SQ8_ERR_LAUNCH; }

// Element (block, pos_in_block, 0) of the paged cache for position p of a row.
__device__ __forceinline__ size_t paged_row(const int32_t* __restrict__ table, int p, int block_size,
                                            int kv_dim) {
  const int block = table[p / block_size];
  return (static_cast<size_t>(block) * block_size + p % block_size) * kv_dim;
}

// One workgroup per row: rotate its q pairs in place, rotate its k pairs and write k and v to the
// row's cache slot.
__global__ __launch_bounds__(kBlock) void paged_rope_kv_kernel(
    float* __restrict__ qkv, int head_num, int kv_head_num, int head_size,
    const int32_t* __restrict__ positions, const int32_t* __restrict__ block_table,
    int table_stride, int block_size, const float* __restrict__ sin_cache,
    const float* __restrict__ cos_cache, float* __restrict__ kcache, float* __restrict__ vcache) {
  const int r = blockIdx.x;
  const int dim = head_num * head_size, kv_dim = kv_head_num * head_size;
  const int half = head_size / 2;
  const int p = positions[r];
  float* row = qkv + static_cast<size_t>(r) * (dim + 2 * kv_dim);
  const size_t slot = paged_row(block_table + static_cast<size_t>(r) * table_stride, p,
                                block_size, kv_dim);
  const float* sn = sin_cache + static_cast<size_t>(p) * head_size;
  const float* cs = cos_cache + static_cast<size_t>(p) * head_size;
  for (int idx = threadIdx.x; idx < (head_num + kv_head_num) * half; idx += kBlock) {
    const int head = idx / half, i = idx % half;
    const float fci = sn[2 * i], fcr = cs[2 * i];
    const int o0 = head * head_size + i, o1 = o0 + half;  // k heads follow the q heads in a row
    const float a = row[o0], b = row[o1];
    const float r0 = fcr * a - fci * b, r1 = fcr * b + fci * a;
    if (head < head_num) {
      row[o0] = r0;
      row[o1] = r1;
    } else {
      const int ko = o0 - dim;
      kcache[slot + ko] = r0;
      kcache[slot + ko + half] = r1;
    }
  }
  for (int d = threadIdx.x; d < kv_dim; d += kBlock) vcache[slot + d] = row[dim + kv_dim + d];
}

// One workgroup (kAttnWaves waves) per (row, query head); the decode attention design with the
// cache rows addressed through the row's block table: wave w owns positions w, w + W, ...; lane l
// holds head dims l, l + 64, ...; scores are wave-reduced dot products and the softmax runs online
// per wave (running max, sum and weighted values), combined across the waves at the end.
template <int HS_MAX>
__global__ __launch_bounds__(kAttnWaves * kWave) void paged_attention_kernel(
    const float* __restrict__ qkv, int q_stride, int head_num, int kv_head_num, int head_size,
    const int32_t* __restrict__ positions, const int32_t* __restrict__ block_table,
    int table_stride, int block_size, const float* kcache, const float* vcache,
    float* __restrict__ out) {
  constexpr int DPL = HS_MAX / kWave;
  constexpr int PCH = 4;
  constexpr int W = kAttnWaves;
  __shared__ float s_m[W], s_l[W];
  __shared__ float s_acc[W][HS_MAX];
  const int id = xcd_grouped_id(head_num / kv_head_num);
  const int r = id / head_num, head = id % head_num;
  const int seq = positions[r] + 1;
  const int kv_dim = kv_head_num * head_size;
  const int hoff = (head * kv_head_num / head_num) * head_size;
  const int32_t* table = block_table + static_cast<size_t>(r) * table_stride;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nmine = wave < seq ? (seq - 1 - wave) / W + 1 : 0;
  const int nch = (nmine + PCH - 1) / PCH;

  float kr[2][PCH][DPL], vr[2][PCH][DPL];
  // Branch-free: positions past the wave's last (and dims past head_size) re-read valid elements
  // and are never used.
  auto load = [&](int b, int c) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < PCH; ++i) {
      const int t = min(wave + (c * PCH + i) * W, seq - 1);
      const size_t base = paged_row(table, t, block_size, kv_dim) + hoff;
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        const int d = min(lane + j * kWave, head_size - 1);
        kr[b][i][j] = kcache[base + d];
        vr[b][i][j] = vcache[base + d];
      }
    }
  };
  if (nch > 0) load(0, 0);

  const float* qrow = qkv + static_cast<size_t>(r) * q_stride + head * head_size;
  float qv[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j)
    qv[j] = lane + j * kWave < head_size ? qrow[lane + j * kWave] : 0.f;
  const float scale = 1.f / sqrtf(static_cast<float>(head_size));
  float m = -INFINITY, l = 0.f, acc[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) acc[j] = 0.f;
  auto chunk = [&](int b, int c) __attribute__((always_inline)) {
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
    for (int i = 0; i < PCH; ++i) {
      if (c * PCH + i < nmine) {
        const float sc = part[i] * scale;
        const float mn = fmaxf(m, sc);
        const float f = expf(m - mn), p = expf(sc - mn);
        l = fmaf(l, f, p);
#pragma unroll
        for (int j = 0; j < DPL; ++j) acc[j] = fmaf(acc[j], f, p * vr[b][i][j]);
        m = mn;
      }
    }
  };
  for (int c = 0; c < nch; c += 2) {
    load(1, min(c + 1, nch - 1));
    chunk(0, c);
    if (c + 1 >= nch) break;
    load(0, min(c + 2, nch - 1));
    chunk(1, c + 1);
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
  float* orow = out + static_cast<size_t>(r) * head_num * head_size + head * head_size;
  for (int d = threadIdx.x; d < head_size; d += W * kWave) {
    float o = 0.f, lt = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float f = s_m[w] == -INFINITY ? 0.f : expf(s_m[w] - mx);
      o = fmaf(s_acc[w][d], f, o);
      lt = fmaf(s_l[w], f, lt);
    }
    orow[d] = o / lt;
  }
}

__global__ __launch_bounds__(kBlock) void swiglu_rows_kernel(const float* __restrict__ gu,
                                                             int ffn, float* __restrict__ out) {
  const float* a = gu + static_cast<size_t>(blockIdx.y) * 2 * ffn;
  float* o = out + static_cast<size_t>(blockIdx.y) * ffn;
  for (int i = blockIdx.x * kBlock + threadIdx.x; i < ffn; i += gridDim.x * kBlock) {
    const float v = a[i];
    const float sig = 1.0f / (1.0f + expf(-v));
    o[i] = (v * sig) * a[ffn + i];
  }
}

__device__ __forceinline__ bool first_max_better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// One workgroup (kArgBlock threads) per row: strided float4 scan keeping the first maximum, then a
// wave and workgroup reduction that prefers the smaller index on ties. NaN never compares greater.
constexpr int kArgBlock = 1024;
__global__ __launch_bounds__(kArgBlock) void argmax_rows_kernel(const float* __restrict__ logits,
                                                                int n, int32_t* __restrict__ out) {
  __shared__ float sv[kArgBlock / kWave];
  __shared__ int si[kArgBlock / kWave];
  const float* row = logits + static_cast<size_t>(blockIdx.x) * n;
  float best = -INFINITY;
  int bi = INT_MAX;
  auto take = [&](float v, int i) __attribute__((always_inline)) {
    if (v > best || (bi == INT_MAX && v == best)) {
      best = v;
      bi = i;
    }
  };
  const bool vec = n % 4 == 0 && (reinterpret_cast<uintptr_t>(row) & 15) == 0;
  if (vec) {
    const float4* r4 = reinterpret_cast<const float4*>(row);
    for (int i = threadIdx.x; i < n / 4; i += kArgBlock) {
      const float4 v = r4[i];
      take(v.x, 4 * i);
      take(v.y, 4 * i + 1);
      take(v.z, 4 * i + 2);
      take(v.w, 4 * i + 3);
    }
  } else {
    for (int i = threadIdx.x; i < n; i += kArgBlock) take(row[i], i);
  }
#pragma unroll
  for (int off = 32; off >= 1; off /= 2) {
    const float ov = __shfl_xor(best, off, kWave);
    const int oi = __shfl_xor(bi, off, kWave);
    if (first_max_better(ov, oi, best, bi)) {
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
    for (int w = 1; w < kArgBlock / kWave; ++w)
      if (first_max_better(sv[w], si[w], best, bi)) {
        best = sv[w];
        bi = si[w];
      }
    out[blockIdx.x] = bi == INT_MAX ? 0 : bi;
  }
}

}  // namespace
}  // namespace sq8

using namespace sq8;

extern "C" {

int sq8_paged_rope_kv(float* qkv, int rows, int head_num, int kv_head_num, int head_size,
                      const int32_t* positions, const int32_t* block_table, int table_stride,
                      int block_size, const float* sin_cache, const float* cos_cache,
                      float* key_cache, float* value_cache, void* hip_stream) {
  if (!qkv || !positions || !block_table || !sin_cache || !cos_cache || !key_cache ||
      !value_cache)
    return SQ8_ERR_NULL;
  if (rows <= 0 || head_num <= 0 || kv_head_num <= 0 || head_num % kv_head_num ||
      head_size <= 0 || head_size % 2 || table_stride <= 0 || block_size <= 0)
    return SQ8_ERR_DIMS;
  hipLaunchKernelGGL(paged_rope_kv_kernel, dim3(rows), dim3(kBlock), 0, stream_of(hip_stream),
                     qkv, head_num, kv_head_num, head_size, positions, block_table, table_stride,
                     block_size, sin_cache, cos_cache, key_cache, value_cache);
  return launched();
}

int sq8_paged_attention(const float* qkv, int q_stride, int rows, int head_num, int kv_head_num,
                        int head_size, const int32_t* positions, const int32_t* block_table,
                        int table_stride, int block_size, const float* key_cache,
                        const float* value_cache, float* out, void* hip_stream) {
  if (!qkv || !positions || !block_table || !key_cache || !value_cache || !out)
    return SQ8_ERR_NULL;
  if (rows <= 0 || head_num <= 0 || kv_head_num <= 0 || head_num % kv_head_num ||
      head_size <= 0 || head_size > 256 || q_stride < head_num * head_size || table_stride <= 0 ||
      block_size <= 0 || static_cast<int64_t>(rows) * head_num > 0x7fffffff)
    return SQ8_ERR_DIMS;
  const dim3 grid(rows * head_num), block(kAttnWaves * kWave);
  if (head_size <= 128)
    hipLaunchKernelGGL((paged_attention_kernel<128>), grid, block, 0, stream_of(hip_stream), qkv,
                       q_stride, head_num, kv_head_num, head_size, positions, block_table,
                       table_stride, block_size, key_cache, value_cache, out);
  else
    hipLaunchKernelGGL((paged_attention_kernel<256>), grid, block, 0, stream_of(hip_stream), qkv,
                       q_stride, head_num, kv_head_num, head_size, positions, block_table,
                       table_stride, block_size, key_cache, value_cache, out);
  return launched();
}

int sq8_swiglu_rows(const float* gate_up, int rows, int ffn, float* out, void* hip_stream) {
  if (!gate_up || !out) return SQ8_ERR_NULL;
  if (rows <= 0 || ffn <= 0 || rows > 65535) return SQ8_ERR_DIMS;
  const int gx = (ffn + kBlock - 1) / kBlock;
  hipLaunchKernelGGL(swiglu_rows_kernel, dim3(gx < 64 ? gx : 64, rows), dim3(kBlock), 0,
                     stream_of(hip_stream), gate_up, ffn, out);
  return launched();
}

int sq8_argmax_rows(const float* logits, int rows, int n, int32_t* out, void* hip_stream) {
  if (!logits || !out) return SQ8_ERR_NULL;
  if (rows <= 0 || n <= 0) return SQ8_ERR_DIMS;
  hipLaunchKernelGGL(argmax_rows_kernel, dim3(rows), dim3(kArgBlock), 0, stream_of(hip_stream),
                     logits, n, out);
  return launched();
}

}  // extern "C"
