// Continuous-batching operators (paged KV cache) for gfx950: rows of different sequences, each at
// its own position, in one launch. C ABI in include/sq8_batch.h.
#include <float.h>
#include <algorithm>
#include <limits.h>
#include <math.h>

#include "sq8.h"
#include "sq8_batch.h"
#include "sq8_common.h"

namespace sq8 {
namespace {

constexpr int kBlock = 256;
#ifndef SQ8_ATTN_WAVES
#define SQ8_ATTN_WAVES 8
#endif
#ifndef SQ8_ATTN_CHUNK
#define SQ8_ATTN_CHUNK 4
#endif
constexpr int kAttnWaves = SQ8_ATTN_WAVES;  // waves per (row, head) attention workgroup
constexpr int kAttnChunk = SQ8_ATTN_CHUNK;  // cache positions per wave per load step
constexpr int kRowU = 2;                   // positions per 16-lane group per step
constexpr int kAttnTableCap = 4096;        // block-table entries staged in LDS by the row kernel
// Split-KV attention (sq8_paged_attention_ws): the work-item target per kv head is
// kAttnFillItems / kv_head_num items when the unsplit grid (rows x kv heads) is below
// kAttnFillUnits workgroups, else rows / kAttnBalanceDiv (chunks of about kAttnBalanceDiv mean
// row lengths: only rows longer than that split); chunks are at least kAttnMinChunk positions.
#ifndef SQ8_ATTN_MIN_CHUNK
#define SQ8_ATTN_MIN_CHUNK 128
#endif
#ifndef SQ8_ATTN_FILL
#define SQ8_ATTN_FILL 768
#endif
#ifndef SQ8_ATTN_BAL
#define SQ8_ATTN_BAL 1
#endif
constexpr int kAttnMinChunk = SQ8_ATTN_MIN_CHUNK;
constexpr int kAttnFillItems = SQ8_ATTN_FILL;  // 3 four-wave workgroups per CU on 256 CUs
constexpr int kAttnFillUnits = 512;
constexpr int kAttnBalanceDiv = SQ8_ATTN_BAL;
constexpr int kAttnSplitMaxRows = 4096;

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
// holds DPL head dims (contiguous, one vector load per cache row, when VEC; else l, l + 64, ...);
// scores are wave-reduced dot products and the softmax runs online per wave (running max, sum
// and weighted values), combined across the waves at the end. kAttnChunk positions per wave are
// loaded per step, and the next step's are in flight while one is used: a row's cache is read
// at memory latency / (waves x chunk) positions, the bound when few rows are long.
template <int HS_MAX, bool VEC>
__global__ __launch_bounds__(kAttnWaves * kWave) void paged_attention_kernel(
    const float* __restrict__ qkv, int q_stride, int head_num, int kv_head_num, int head_size,
    const int32_t* __restrict__ positions, const int32_t* __restrict__ block_table,
    int table_stride, int block_size, const float* kcache, const float* vcache,
    float* __restrict__ out) {
  constexpr int DPL = HS_MAX / kWave;
  constexpr int PCH = kAttnChunk;
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
  // Head dim j of this lane, and the first dim it loads (clamped into the head: lanes past
  // head_size load valid elements and are never used).
  auto dim = [&](int j) __attribute__((always_inline)) {
    return VEC ? DPL * lane + j : lane + j * kWave;
  };
  const int d0 = VEC ? min(DPL * lane, head_size - DPL) : 0;

  float kr[2][PCH][DPL], vr[2][PCH][DPL];
  // Branch-free: positions past the wave's last re-read valid elements and are never used.
  auto load = [&](int b, int c) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < PCH; ++i) {
      const int t = min(wave + (c * PCH + i) * W, seq - 1);
      const size_t base = paged_row(table, t, block_size, kv_dim) + hoff;
      if constexpr (VEC && DPL == 2) {
        const float2 k2 = *reinterpret_cast<const float2*>(kcache + base + d0);
        const float2 v2 = *reinterpret_cast<const float2*>(vcache + base + d0);
        kr[b][i][0] = k2.x;
        kr[b][i][1] = k2.y;
        vr[b][i][0] = v2.x;
        vr[b][i][1] = v2.y;
      } else if constexpr (VEC && DPL == 4) {
        const float4 k4 = *reinterpret_cast<const float4*>(kcache + base + d0);
        const float4 v4 = *reinterpret_cast<const float4*>(vcache + base + d0);
        kr[b][i][0] = k4.x;
        kr[b][i][1] = k4.y;
        kr[b][i][2] = k4.z;
        kr[b][i][3] = k4.w;
        vr[b][i][0] = v4.x;
        vr[b][i][1] = v4.y;
        vr[b][i][2] = v4.z;
        vr[b][i][3] = v4.w;
      } else {
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const int d = min(dim(j), head_size - 1);
          kr[b][i][j] = kcache[base + d];
          vr[b][i][j] = vcache[base + d];
        }
      }
    }
  };
  if (nch > 0) load(0, 0);

  const float* qrow = qkv + static_cast<size_t>(r) * q_stride + head * head_size;
  float qv[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) qv[j] = dim(j) < head_size ? qrow[dim(j)] : 0.f;
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
    if (dim(j) < head_size) s_acc[wave][dim(j)] = acc[j];
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

// Sum of v over the 16 lanes of each DPP row (lanes 16k .. 16k+15); every lane gets the sum.
// quad_perm [1,0,3,2] and [2,3,0,1] sum each quad, row_half_mirror adds the other quad of the
// half-row and row_mirror the other half: all VALU, no LDS permute.
__device__ __forceinline__ float row16_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  return v;
}

// One workgroup (W waves) per (row, kv head), for the G query heads that read the kv
// head. Each 16-lane group of a wave owns one cache position at a time and lane li of the group
// holds head dims DPL*li .. +DPL-1 (one coalesced 16*DPL-float row per group and load); a wave
// steps over kRowStep positions (kRowU per group), the next step's rows in flight while one is
// used. A score is a 16-lane DPP sum; each 16-lane group keeps its own running max per head,
// updated once per step from the group's U scores, so a (position, head) costs DPL FMAs, 4 DPP
// adds and one exponential and a step needs no cross-group exchange (a wave-wide max per step,
// through two lane permutes per head, made every step wait on the permute latency). Groups are
// brought to a common max and summed at the end, then the waves are combined.
//
// With n_target > 0 (split KV, the flash-decoding split of paged_kernels.cu:96-294) the rows'
// positions are cut into chunks of C = max(kAttnMinChunk, ceil(T / n_target)) positions, T the
// total over all rows, so a row of n positions makes ceil(n / C) work items and there are at most
// n_target + rows of them per kv head; blockIdx.x / kv_head_num picks a work item (items numbered
// row by row) and a workgroup past the last item exits at once. A row of one chunk writes its
// output directly. Otherwise each chunk stores its un-normalised head outputs, max and sum to
// part (agent-scope stores, released before the ticket), takes a ticket per (row, kv head),
// and the chunk that finishes last merges the row's chunks and resets the ticket to zero.
template <int DPL, int GMAX, int W>
__global__ __launch_bounds__(W * kWave) void paged_attention_rows_kernel(
    const float* __restrict__ qkv, int q_stride, int head_num, int kv_head_num, int head_size,
    const int32_t* __restrict__ positions, const int32_t* __restrict__ block_table,
    int table_stride, int block_size, const float* kcache, const float* vcache,
    float* __restrict__ out, int rows, int n_target, float* __restrict__ part,
    unsigned* __restrict__ tickets) {
  constexpr int U = kRowU;
  constexpr int SP = 4 * U;  // positions per wave per step
  constexpr int HS = 16 * DPL;
  constexpr int NV = DPL / 4;  // float4 per lane per cache row
  __shared__ float s_m[W][GMAX], s_l[W][GMAX];
  __shared__ float s_acc[W][GMAX][HS];
  __shared__ int32_t table[kAttnTableCap];  // the row's block table (table_stride <= cap)
  __shared__ int s_item[3];                 // split KV: row, its first item, chunk length
  const int G = head_num / kv_head_num;
  const int item = blockIdx.x / kv_head_num, kvh = blockIdx.x % kv_head_num;
  int r = item, first = item, chunk = 0;
  if (n_target > 0) {
    if (threadIdx.x < kWave) {  // wave 0 finds the work item's row and chunk
      const int ln = threadIdx.x;
      int t = 0;
      for (int i = ln; i < rows; i += kWave) t += positions[i] + 1;
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) t += __shfl_xor(t, d, kWave);
      const int c = max(kAttnMinChunk, t / n_target + (t % n_target != 0));  // t may be INT_MAX
      int base = 0, sel = -1, sel_first = 0;
      for (int i0 = 0; i0 < rows; i0 += kWave) {
        const int i = i0 + ln;
        const int n = i < rows ? (positions[i] + c) / c : 0;  // ceil(row length / c)
        int incl = n;
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
          const int v = __shfl_up(incl, d, kWave);
          if (ln >= d) incl += v;
        }
        const int excl = base + incl - n;
        const uint64_t hit = __ballot(n > 0 && item >= excl && item < base + incl);
        if (hit) {
          const int src = __builtin_ctzll(hit);
          sel = __shfl(i, src, kWave);
          sel_first = __shfl(excl, src, kWave);
          break;
        }
        base += __shfl(incl, kWave - 1, kWave);
      }
      if (ln == 0) {
        s_item[0] = sel;
        s_item[1] = sel_first;
        s_item[2] = c;
      }
    }
    __syncthreads();
    r = s_item[0];
    first = s_item[1];
    chunk = s_item[2];
    if (r < 0) return;  // uniform across the workgroup
  }
  const int row_len = positions[r] + 1;
  const int p0 = chunk > 0 ? (item - first) * chunk : 0;
  const int nchunks = chunk > 0 ? (row_len + chunk - 1) / chunk : 1;
  // Positions below are relative to the first table block of the range, b0 * block_size.
  const int b0 = p0 / block_size, pbase = p0 - b0 * block_size;
  const int seq = min(row_len, chunk > 0 ? p0 + chunk : row_len) - p0;  // positions in range
  const int kv_dim = kv_head_num * HS, hoff = kvh * HS;
  // Stage the range's block-table entries once: every cache-row address then costs an LDS read
  // instead of a dependent global load ahead of each step's key/value loads.
  {
    const int32_t* gt = block_table + static_cast<size_t>(r) * table_stride + b0;
    const int nb = (pbase + seq + block_size - 1) / block_size;
    for (int i = threadIdx.x; i < nb; i += W * kWave) table[i] = gt[i];
    __syncthreads();
  }
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = lane >> 4, li = lane & 15;
  const int nsteps = (seq + SP - 1) / SP;
  const int nmine = wave < nsteps ? (nsteps - 1 - wave) / W + 1 : 0;

  float4 kb[2][U][NV], vb[2][U][NV];
  // Position of group grp's u-th row at the wave's c-th step (re-reads position seq - 1 past the
  // end; such scores are masked).
  auto posn = [&](int c, int u) __attribute__((always_inline)) {
    return (c * W + wave) * SP + u * 4 + grp;
  };
  auto load = [&](int b, int c) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const size_t base =
          paged_row(table, pbase + min(posn(c, u), seq - 1), block_size, kv_dim) + hoff +
          DPL * li;
#pragma unroll
      for (int i = 0; i < NV; ++i) {
        kb[b][u][i] = *reinterpret_cast<const float4*>(kcache + base + 4 * i);
        vb[b][u][i] = *reinterpret_cast<const float4*>(vcache + base + 4 * i);
      }
    }
  };
  if (nmine > 0) load(0, 0);

  const float scale = 1.f / sqrtf(static_cast<float>(HS));
  const float* qrow = qkv + static_cast<size_t>(r) * q_stride + kvh * G * HS + DPL * li;
  float q[GMAX][DPL], m[GMAX], l[GMAX], acc[GMAX][DPL];
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.f;
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      q[g][j] = g < G ? qrow[g * HS + j] * scale : 0.f;
      acc[g][j] = 0.f;
    }
  }
  auto step = [&](int b, int c) __attribute__((always_inline)) {
#pragma unroll
    for (int g = 0; g < GMAX; ++g) {
      if (g >= G) break;
      float s[U], mx = -INFINITY;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          a = fmaf(q[g][4 * i], kb[b][u][i].x, a);
          a = fmaf(q[g][4 * i + 1], kb[b][u][i].y, a);
          a = fmaf(q[g][4 * i + 2], kb[b][u][i].z, a);
          a = fmaf(q[g][4 * i + 3], kb[b][u][i].w, a);
        }
        const float sum = row16_sum(a);  // all lanes of the row take part
        s[u] = posn(c, u) < seq ? sum : -INFINITY;
        mx = fmaxf(mx, s[u]);
      }
      // Each 16-lane group keeps its own running max (no cross-group exchange per step); a
      // group whose positions so far are all past the sequence end still has max -inf.
      const float mn = fmaxf(m[g], mx);
      const bool none = mn == -INFINITY;
      const float f = none ? 1.f : expf(m[g] - mn);
      l[g] *= f;
#pragma unroll
      for (int j = 0; j < DPL; ++j) acc[g][j] *= f;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float p = none ? 0.f : expf(s[u] - mn);
        l[g] += p;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
          acc[g][4 * i] = fmaf(p, vb[b][u][i].x, acc[g][4 * i]);
          acc[g][4 * i + 1] = fmaf(p, vb[b][u][i].y, acc[g][4 * i + 1]);
          acc[g][4 * i + 2] = fmaf(p, vb[b][u][i].z, acc[g][4 * i + 2]);
          acc[g][4 * i + 3] = fmaf(p, vb[b][u][i].w, acc[g][4 * i + 3]);
        }
      }
      m[g] = mn;
    }
  };
  for (int c = 0; c < nmine; c += 2) {
    load(1, min(c + 1, nmine - 1));
    step(0, c);
    if (c + 1 >= nmine) break;
    load(0, min(c + 2, nmine - 1));
    step(1, c + 1);
  }

  // Bring the 4 groups to the wave's max and sum them, then combine the waves.
#pragma unroll
  for (int g = 0; g < GMAX; ++g) {
    if (g >= G) break;
    float mw = fmaxf(m[g], __shfl_xor(m[g], 16, kWave));
    mw = fmaxf(mw, __shfl_xor(mw, 32, kWave));
    const float gscale = m[g] == -INFINITY ? 0.f : expf(m[g] - mw);
    m[g] = mw;
    l[g] *= gscale;
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[g][j] *= gscale;
    float lt = l[g];
    lt += __shfl_xor(lt, 16, kWave);
    lt += __shfl_xor(lt, 32, kWave);
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      float a = acc[g][j];
      a += __shfl_xor(a, 16, kWave);
      a += __shfl_xor(a, 32, kWave);
      acc[g][j] = a;
    }
    if (lane == 0) {
      s_m[wave][g] = m[g];
      s_l[wave][g] = lt;
    }
    if (grp == 0) {
#pragma unroll
      for (int j = 0; j < DPL; ++j) s_acc[wave][g][DPL * li + j] = acc[g][j];
    }
  }
  __syncthreads();
  // Partials of (row, kv head) chunk c: G head outputs of HS floats, then G maxima, then G sums.
  const int pstride = G * (HS + 2);
  const size_t pitem = static_cast<size_t>(kv_head_num) * pstride;  // floats per work item
  float* const pbuf = part + (static_cast<size_t>(first) * kv_head_num + kvh) * pstride;
  for (int e = threadIdx.x; e < G * HS; e += W * kWave) {
    const int g = e / HS, d = e % HS;
    float mx = s_m[0][g];
#pragma unroll
    for (int w = 1; w < W; ++w) mx = fmaxf(mx, s_m[w][g]);
    float o = 0.f, lt = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float f = s_m[w][g] == -INFINITY ? 0.f : expf(s_m[w][g] - mx);
      o = fmaf(s_acc[w][g][d], f, o);
      lt = fmaf(s_l[w][g], f, lt);
    }
    if (nchunks == 1) {
      out[(static_cast<size_t>(r) * head_num + kvh * G + g) * HS + d] = o / lt;
    } else {
      float* const c = pbuf + static_cast<size_t>(item - first) * pitem;
      __hip_atomic_store(c + e, o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (d == 0) {
        __hip_atomic_store(c + G * HS + g, mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(c + G * HS + G + g, lt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if (nchunks == 1) return;
  publish_partials();
  __shared__ bool is_last;
  __syncthreads();
  if (threadIdx.x == 0)
    is_last = __hip_atomic_fetch_add(&tickets[r * kv_head_num + kvh], 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT) ==
              static_cast<unsigned>(nchunks - 1);
  __syncthreads();
  if (!is_last) return;
  acquire_partials();
  // Merge in batches of kMergeBatch chunks, every load of a batch issued before any is used (one
  // memory latency per batch, not per chunk), with a running max across batches.
  constexpr int kMergeBatch = 8;
  for (int e = threadIdx.x; e < G * HS; e += W * kWave) {
    const int g = e / HS, d = e % HS;
    float mx = -INFINITY, o = 0.f, lt = 0.f;
    for (int c0 = 0; c0 < nchunks; c0 += kMergeBatch) {
      float mv[kMergeBatch], lv[kMergeBatch], ov[kMergeBatch];
#pragma unroll
      for (int k = 0; k < kMergeBatch; ++k) {
        const float* const pc = pbuf + static_cast<size_t>(min(c0 + k, nchunks - 1)) * pitem;
        mv[k] = __hip_atomic_load(pc + G * HS + g, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        lv[k] = __hip_atomic_load(pc + G * HS + G + g, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
        ov[k] = __hip_atomic_load(pc + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      // Chunks past the row's last repeat the last chunk and are skipped; every chunk has at
      // least one position, so its max is finite.
      float bm = mx;
#pragma unroll
      for (int k = 0; k < kMergeBatch; ++k)
        if (c0 + k < nchunks) bm = fmaxf(bm, mv[k]);
      const float f0 = mx == -INFINITY ? 0.f : expf(mx - bm);
      o *= f0;
      lt *= f0;
#pragma unroll
      for (int k = 0; k < kMergeBatch; ++k) {
        if (c0 + k < nchunks) {
          const float f = expf(mv[k] - bm);
          o = fmaf(ov[k], f, o);
          lt = fmaf(lv[k], f, lt);
        }
      }
      mx = bm;
    }
    out[(static_cast<size_t>(r) * head_num + kvh * G + g) * HS + d] = o / lt;
  }
  if (threadIdx.x == 0)
    __hip_atomic_store(&tickets[r * kv_head_num + kvh], 0u, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
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

// Shapes the (row, kv head) kernel covers.
bool rows_kernel_fits(int head_size, int G) {
  return (head_size == 128 || head_size == 64) && G <= 8;
}
// Work-item target per kv head of split-KV attention (0: no split).
int split_target(int rows, int kv_head_num, int table_stride, int block_size) {
  // The kernel sums the rows' lengths (each at most table_stride * block_size) in 32 bits.
  const int64_t span = static_cast<int64_t>(table_stride) * block_size;
  if (rows > kAttnSplitMaxRows || table_stride >= kAttnTableCap || span <= kAttnMinChunk ||
      span * rows > INT_MAX)
    return 0;
  const int64_t units = static_cast<int64_t>(rows) * kv_head_num;
  const int fill = units < kAttnFillUnits ? (kAttnFillItems + kv_head_num - 1) / kv_head_num : 0;
  return max(max(fill, rows / kAttnBalanceDiv), 1);
}
// Ticket area at the start of the split-KV workspace: one per (row, kv head) for every row count
// that can split, 256-byte aligned. Its size depends on kv_head_num only, so calls of different
// row counts sharing one workspace agree on where the tickets end and the partials begin (a
// smaller call's partials never land on a larger call's tickets).
int64_t ticket_bytes(int kv_head_num) {
  return (static_cast<int64_t>(kAttnSplitMaxRows) * kv_head_num * 4 + 255) / 256 * 256;
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
  return sq8_paged_attention_ws(qkv, q_stride, rows, head_num, kv_head_num, head_size, positions,
                                block_table, table_stride, block_size, key_cache, value_cache,
                                out, nullptr, 0, hip_stream);
}

size_t sq8_paged_attention_workspace_bytes(int rows, int head_num, int kv_head_num,
                                           int head_size, int table_stride, int block_size) {
  if (rows <= 0 || head_num <= 0 || kv_head_num <= 0 || head_num % kv_head_num ||
      table_stride <= 0 || block_size <= 0)
    return 0;
  const int G = head_num / kv_head_num;
  if (!rows_kernel_fits(head_size, G)) return 0;
  // Enough for every call of at most `rows` rows (the item count is not monotone in rows: small
  // batches fill the GPU with more items).
  int64_t items = 0;
  for (int n = 1; n <= std::min(rows, kAttnSplitMaxRows); ++n) {
    const int t = split_target(n, kv_head_num, table_stride, block_size);
    if (t > 0) items = std::max<int64_t>(items, t + n);
  }
  if (items == 0) return 0;
  return static_cast<size_t>(ticket_bytes(kv_head_num) +
                             items * kv_head_num * G * (head_size + 2) * 4);
}

int sq8_paged_attention_ws(const float* qkv, int q_stride, int rows, int head_num,
                           int kv_head_num, int head_size, const int32_t* positions,
                           const int32_t* block_table, int table_stride, int block_size,
                           const float* key_cache, const float* value_cache, float* out,
                           void* workspace, size_t workspace_bytes, void* hip_stream) {
  if (!qkv || !positions || !block_table || !key_cache || !value_cache || !out)
    return SQ8_ERR_NULL;
  if (rows <= 0 || head_num <= 0 || kv_head_num <= 0 || head_num % kv_head_num ||
      head_size <= 0 || head_size > 256 || q_stride < head_num * head_size || table_stride <= 0 ||
      block_size <= 0 || static_cast<int64_t>(rows) * head_num > 0x7fffffff)
    return SQ8_ERR_DIMS;
  const hipStream_t st = stream_of(hip_stream);
  const int G = head_num / kv_head_num;
  const bool k16 = reinterpret_cast<uintptr_t>(key_cache) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(value_cache) % 16 == 0;
  const size_t need = sq8_paged_attention_workspace_bytes(rows, head_num, kv_head_num, head_size,
                                                          table_stride, block_size);
  if (need > 0 && workspace && workspace_bytes < need) return SQ8_ERR_WORKSPACE;
  const bool split = need > 0 && workspace != nullptr && k16;
  if (rows_kernel_fits(head_size, G) && k16 &&
      (split || table_stride <= kAttnTableCap)) {
    // Unsplit with few workgroups (few, typically long, rows): 8 waves each to keep more rows
    // in flight. Split: a workgroup of 4 waves per work item.
    const int64_t units = static_cast<int64_t>(rows) * kv_head_num;
    const bool wide = !split && units < 2 * cu_count();
    const int target = split ? split_target(rows, kv_head_num, table_stride, block_size) : 0;
    unsigned* tickets = split ? static_cast<unsigned*>(workspace) : nullptr;
    float* part = split ? reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                                   ticket_bytes(kv_head_num))
                        : nullptr;
    const dim3 grid((rows + target) * kv_head_num), block((wide ? 8 : 4) * kWave);
    const auto rk = [&](auto kernel) {
      hipLaunchKernelGGL(kernel, grid, block, 0, st, qkv, q_stride, head_num, kv_head_num,
                         head_size, positions, block_table, table_stride, block_size, key_cache,
                         value_cache, out, rows, target, part, tickets);
    };
    if (head_size == 64)
      wide ? rk(paged_attention_rows_kernel<4, 8, 8>) : rk(paged_attention_rows_kernel<4, 8, 4>);
    else if (G <= 4)
      wide ? rk(paged_attention_rows_kernel<8, 4, 8>) : rk(paged_attention_rows_kernel<8, 4, 4>);
    else
      wide ? rk(paged_attention_rows_kernel<8, 8, 8>) : rk(paged_attention_rows_kernel<8, 8, 4>);
    return launched();
  }
  const dim3 grid(rows * head_num), block(kAttnWaves * kWave);
  // One vector load per cache row when every lane's dims are contiguous and aligned.
  const int dpl = head_size <= 128 ? 2 : 4;
  const bool vec = head_size % dpl == 0 && kv_head_num * head_size % dpl == 0 &&
                   reinterpret_cast<uintptr_t>(key_cache) % (4 * dpl) == 0 &&
                   reinterpret_cast<uintptr_t>(value_cache) % (4 * dpl) == 0;
  const auto args = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, block, 0, st, qkv, q_stride, head_num, kv_head_num, head_size,
                       positions, block_table, table_stride, block_size, key_cache, value_cache,
                       out);
  };
  if (head_size <= 128)
    vec ? args(paged_attention_kernel<128, true>) : args(paged_attention_kernel<128, false>);
  else
    vec ? args(paged_attention_kernel<256, true>) : args(paged_attention_kernel<256, false>);
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
