// MFMA kernels for token counts above the GEMV range (small-batch decode and prefill), gfx950.
//
// Reference behaviour replaced: matmul_kernel_cu_fp32int8<128> (matmul_kernel.cu:65-99) computes
// y[b, n] = sum_k x[b, k] * scale * (float)w[n, k] with fp32 CUDA-core arithmetic, re-reading each
// weight row once per batch row. Here the product runs on the matrix cores:
//
//  * Activations: fp32 cannot feed an f16 MFMA exactly, so each token row is split once into
//    x * 2^e = hi + lo with hi = f16(x * 2^e) and lo = f16(x * 2^e - hi). The power of two 2^e puts
//    the row's absmax in [2^13, 2^14), far from f16 overflow, and makes hi + lo carry ~22 bits,
//    about fp32's precision (split_x_kernel). The output is multiplied back by 2^-e exactly.
//  * Weights: int8 is exact in f16. A 16-byte chunk is biased to unsigned (xor 0x80), interleaved
//    with the f16 exponent byte 0x64 by v_perm (giving 1024 + 128 + q), and one packed f16 add of
//    -1152 yields q exactly: two VALU ops per 4 weights.
//  * One K step of the main loop is one 64-wide weight group. Its partial product P (hi and lo
//    MFMAs chained in fp32) is formed from zero, then acc += scale[n, g] * P with one FMA per
//    output: the per-group scale never touches the weights, so no rounding is added on that side.
//  * v_mfma_f32_32x32x16_f16 tiles; a workgroup of 4 or 8 waves owns a 64 x 256 or 128 x 256
//    output tile and streams its operands through a 3-deep ring of LDS stages filled by direct
//    global -> LDS DMA (gemm_kernel below), one barrier per group.
//  * Skinny shapes (few tokens, few output tiles) split K over gridDim.z; partial tiles go to the
//    workspace and a second kernel sums them in split order (deterministic).
#include <algorithm>
#include <type_traits>

#include "sq8_common.h"

namespace sq8 {

namespace {

constexpr int kThreads = 256;
constexpr int LDS_STRIDE = 72;  // halves per staged row (64 + 8 padding against bank conflicts)

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- activation split
// Threads and register-held float4 per thread of the row-split kernels: a row of up to
// kSplitThreads * 4 * kSplitV values is read once, kept in registers while the workgroup finds
// its absmax, and converted from there (one memory round trip); longer rows are read twice.
constexpr int kSplitThreads = 512;
constexpr int kSplitV = 8;

// Power of two for a row of absmax `amax`: x * 2^e has its absmax in [2^13, 2^14).
__device__ __forceinline__ int row_exponent(float amax) {
  int e = 0;
  if (amax > 0.f && amax <= 3.402823466e38f) {
    int ex;
    frexpf(amax, &ex);  // amax = f * 2^ex, f in [0.5, 1)
    e = min(max(14 - ex, -126), 126);
  }
  return e;
}

__device__ __forceinline__ float absmax4(float4 v) {
  return fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
}

// Load a row (zeros when !live) and return its exponent; v holds the first kSplitV float4 of
// the thread (k = (tid + i * kSplitThreads) * 4) when the row fits, else it is re-read later.
__device__ __forceinline__ int load_row_exponent(const float* __restrict__ xr, int K, bool live,
                                                 float4 (&v)[kSplitV], float* red) {
  const int tid = threadIdx.x;
  const bool regs = K <= kSplitThreads * 4 * kSplitV;
  float amax = 0.f;
  if (regs) {
#pragma unroll
    for (int i = 0; i < kSplitV; ++i) {
      const int k = (tid + i * kSplitThreads) * 4;
      v[i] = live && k < K ? *reinterpret_cast<const float4*>(xr + k)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int i = 0; i < kSplitV; ++i) amax = fmaxf(amax, absmax4(v[i]));
  } else if (live) {
    for (int k = tid * 4; k < K; k += kSplitThreads * 4)
      amax = fmaxf(amax, absmax4(*reinterpret_cast<const float4*>(xr + k)));
  }
#pragma unroll
  for (int off = 32; off >= 1; off /= 2) amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
  if ((tid & (kWave - 1)) == 0) red[tid >> 6] = amax;
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int w = 1; w < kSplitThreads / kWave; ++w) amax = fmaxf(amax, red[w]);
  return row_exponent(amax);
}

// Visit the row's float4 chunks with their start k: from registers when the row fits, else
// re-read (zeros when !live).
template <typename F>
__device__ __forceinline__ void for_row_chunks(const float* __restrict__ xr, int K, bool live,
                                               const float4 (&v)[kSplitV], F&& f) {
  const int tid = threadIdx.x;
  if (K <= kSplitThreads * 4 * kSplitV) {
#pragma unroll
    for (int i = 0; i < kSplitV; ++i) {
      const int k = (tid + i * kSplitThreads) * 4;
      if (k < K) f(k, v[i]);
    }
  } else {
    for (int k = tid * 4; k < K; k += kSplitThreads * 4)
      f(k, live ? *reinterpret_cast<const float4*>(xr + k) : make_float4(0.f, 0.f, 0.f, 0.f));
  }
}

// x * 2^e = hi + lo for four values.
__device__ __forceinline__ void split4(float4 v, int e, _Float16 (&h)[4], _Float16 (&l)[4]) {
  const float a[4] = {ldexpf(v.x, e), ldexpf(v.y, e), ldexpf(v.z, e), ldexpf(v.w, e)};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    h[i] = static_cast<_Float16>(a[i]);
    l[i] = static_cast<_Float16>(a[i] - static_cast<float>(h[i]));
  }
}

// One workgroup per token row: absmax, exponent, then hi/lo halves.
__global__ __launch_bounds__(kSplitThreads) void split_x_kernel(const float* __restrict__ x,
                                                              _Float16* __restrict__ xh,
                                                              _Float16* __restrict__ xl,
                                                              float* __restrict__ rscale, int K) {
  __shared__ float red[kSplitThreads / kWave];
  const int m = blockIdx.x;
  const float* xr = x + static_cast<size_t>(m) * K;
  float4 v[kSplitV];
  const int e = load_row_exponent(xr, K, true, v, red);
  if (threadIdx.x == 0) rscale[m] = ldexpf(1.f, -e);
  _Float16* hr = xh + static_cast<size_t>(m) * K;
  _Float16* lr = xl + static_cast<size_t>(m) * K;
  for_row_chunks(xr, K, true, v, [&](int k, float4 c) {
    _Float16 h[4], l[4];
    split4(c, e, h, l);
    *reinterpret_cast<uint2*>(hr + k) = *reinterpret_cast<const uint2*>(h);
    *reinterpret_cast<uint2*>(lr + k) = *reinterpret_cast<const uint2*>(l);
  });
}

// 4 int8 (one dword) -> 4 exact f16 (two dwords), see file comment.
__device__ __forceinline__ void i8x4_to_h4(uint32_t d, uint32_t& lo, uint32_t& hi) {
  const uint32_t u = d ^ 0x80808080u;
  const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
  const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
  const h2 bias = {static_cast<_Float16>(-1152.f), static_cast<_Float16>(-1152.f)};
  h2 ha = __builtin_bit_cast(h2, a) + bias;
  h2 hb = __builtin_bit_cast(h2, b) + bias;
  lo = __builtin_bit_cast(uint32_t, ha);
  hi = __builtin_bit_cast(uint32_t, hb);
}

// ---------------------------------------------------------------- pipelined GEMM (LDS DMA)
// Same arithmetic as mfma_gemm_kernel (hi/lo activation MFMAs per 64-wide group, acc += scale * P),
// fed by a STAGES-deep ring of LDS stages that global_load_lds_dwordx4 fills straight from memory:
// no register staging, so several groups of loads are in flight per wave while the MFMAs run.
//  * Stage layout: x hi [BM][64] f16, x lo [BM][64] f16, w [BN][64] int8 (converted to f16 after
//    the LDS read), scales [BN] fp32 (stored twice per 32 columns, see below).
//  * A DMA instruction writes lane i's 16 bytes to LDS slot base + 16 * i, so the layout is chosen
//    by which global chunk each lane fetches. Chunks are XOR-swizzled within a row so that the
//    MFMA operand reads (32 rows x one 16-byte chunk per instruction) hit distinct banks:
//    x row r keeps chunk c at slot c ^ fx(r), w row r keeps chunk q at slot q ^ fw(r).
//  * The loads are issued from inline asm, so the compiler does not count them; every thread
//    issues the same number per stage (LOADS), and before reading stage s a thread waits until at
//    most (STAGES - 2) stages of its own loads are outstanding, then a barrier publishes all
//    threads' loads. The same barrier tells every wave that the stage being refilled next has
//    been read by all waves. One barrier per 64-wide group.
// GPS groups per stage: x rows of 8*GPS chunks, w rows of 4*GPS chunks.
using ix::swz_w;
using ix::swz_x;

// One 16-byte global -> LDS copy per lane: lane i writes LDS [lds_base + 16 i]. m0 (the LDS
// base register of the DMA) is saved and restored around the copy.
__device__ __forceinline__ void dma16(const void* base, uint32_t voff, uint32_t lds_base) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dwordx4 %2, %3\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds_base), "v"(voff), "s"(base)
      : "memory");
}
__device__ __forceinline__ void dma4(const void* base, uint32_t voff, uint32_t lds_base) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dword %2, %3\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds_base), "v"(voff), "s"(base)
      : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  // gfx9 s_waitcnt encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Output tile (bx, by, bz) of the GEMM's hardware workgroup id: XCD-banded order (ix::gemm_tile).
__device__ __forceinline__ void gemm_tile_coords(int& bx, int& by, int& bz) {
  const ix::Tile3 t = ix::gemm_tile(blockIdx.x, blockIdx.y, blockIdx.z, gridDim.x, gridDim.y,
                                    gridDim.z, SQ8_GEMM_GM);
  bx = t.x, by = t.y, bz = t.z;
}

template <int WAVES_M, int WAVES_N, int TM, int TN, int STAGES, int GPS>
__global__ __launch_bounds__(WAVES_M * WAVES_N * kWave) void gemm_kernel(
    const _Float16* xh, const _Float16* xl, const float* __restrict__ rscale, const int8_t* w,
    const float* s, float* out, int M, int N, int K, int gs, int groups_per_split, Epi epi,
    int pk) {
  using T = PTile<WAVES_M, WAVES_N, TM, TN, STAGES, GPS>;
  static_assert(TN % 2 == 0, "SwiGLU pairs tile j (gate) with tile j + TN/2 (up) of a wave");
  constexpr int HT = TN / 2;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  int bx, by, bz;
  gemm_tile_coords(bx, by, bz);
  const int n0 = bx * T::BN, m0 = by * T::BM;
  const int nsteps = K / T::KB;  // stages of GPS groups; the split is in stages
  const int st_begin = bz * groups_per_split;
  const int st_end = min(nsteps, st_begin + groups_per_split);
  const int gpr = K / gs;
  // Weight row behind tile column c (0 <= c < BN). SwiGLU: the workgroup owns features
  // f0 .. f0 + BN/2 - 1 of F = N/2; a wave's 32-column tiles j < TN/2 hold the gate rows of its
  // features and tiles j + TN/2 their up rows (F rows further on), so one lane holds both halves
  // of each output.
  const bool swiglu = epi.mode == kEpiSwiglu;
  const int F = N / 2, f0 = bx * (T::BN / 2);
  auto feat = [&](int c) __attribute__((always_inline)) { return ix::gemm_feat(c, bx, T::BN, TN); };
  auto wrow = [&](int c) __attribute__((always_inline)) {
    return ix::gemm_row(c, bx, T::BN, TN, N, swiglu);
  };
  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem));

  // Per-thread DMA sources (byte offsets; the K offset of a stage is added to the base pointer).
  uint32_t xoff[T::XL], woff[T::WL], soff[T::SL];
#pragma unroll
  for (int i = 0; i < T::XL; ++i) {
    const int slot = (i * T::NW + wave) * kWave + lane;
    const int r = slot / T::CX, c = (slot % T::CX) ^ swz_x<GPS>(slot / T::CX);
    xoff[i] = static_cast<uint32_t>(min(m0 + r, M - 1)) * K * 2u + c * 16u;
  }
#pragma unroll
  for (int i = 0; i < T::WL; ++i) {
    const int slot = (i * T::NW + wave) * kWave + lane;
    const int r = slot / T::CW, q = (slot % T::CW) ^ swz_w<GPS>(slot / T::CW);
    const uint32_t n = static_cast<uint32_t>(wrow(r));
    // Packed: chunk q of the stage is chunk q % 4 of its group q / 4, in the row's tile block.
    woff[i] = ix::gemm_woff(pk, n, K, q);
  }
#pragma unroll
  for (int i = 0; i < T::SL; ++i) {
    const int run = (i * T::NW + wave) % (T::BN / 32);  // 32-column run of this instruction
    const int c = run * 32 + (lane & 31);
    soff[i] = static_cast<uint32_t>(wrow(c)) * gpr * 4u;
  }
  auto issue = [&](int st, int buf) __attribute__((always_inline)) {
    const uint32_t sb = lds0 + buf * T::STAGE;
    const char* xhb = reinterpret_cast<const char*>(xh) + static_cast<size_t>(st) * T::KB * 2;
    const char* xlb = reinterpret_cast<const char*>(xl) + static_cast<size_t>(st) * T::KB * 2;
    const char* wb = reinterpret_cast<const char*>(w) +
                     static_cast<size_t>(st) * ix::gemm_stage_wstep(pk, GPS);
#pragma unroll
    for (int i = 0; i < T::XL; ++i) {
      const uint32_t d = ((i * T::NW + wave) * kWave) * 16;
      dma16(xhb, xoff[i], sb + d);
      dma16(xlb, xoff[i], sb + T::XB + d);
    }
#pragma unroll
    for (int i = 0; i < T::WL; ++i)
      dma16(wb, woff[i], sb + 2 * T::XB + ((i * T::NW + wave) * kWave) * 16);
#pragma unroll
    for (int i = 0; i < T::SL; ++i) {
      const int g = st * GPS + (i * T::NW + wave) / (T::BN / 32);  // group of this instruction
      const int sg = gs == BK ? g : g * BK / gs;                    // its scale column
      dma4(reinterpret_cast<const char*>(s) + static_cast<size_t>(sg) * 4, soff[i],
           sb + 2 * T::XB + T::WB + (i * T::NW + wave) * 256);
    }
  };

  f16v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // Lane's LDS read offsets inside a stage.
  const int lrow = lane & 31, half = lane >> 5;
  int aoff[TM], boff[TN], scoff[TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int r = (wm * TM + i) * 32 + lrow;
    // chunk (group gi, step t) of the lane: aoff ^ (16 (8 gi + t))
    aoff[i] = r * (T::CX * 16) + ((half * 4) ^ swz_x<GPS>(r)) * 16;
  }
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int r = (wn * TN + j) * 32 + lrow;
    // chunk (group gi, half u): boff ^ (16 (4 gi + u))
    boff[j] = 2 * T::XB + r * (T::CW * 16) + ((half * 2) ^ swz_w<GPS>(r)) * 16;
    scoff[j] = 2 * T::XB + T::WB + (r >> 5) * 256 + (r & 31) * 4;
  }

  if (st_begin < st_end) {
#pragma unroll
    for (int p = 0; p < STAGES - 1; ++p) issue(min(st_begin + p, st_end - 1), p);
  }
  // Wait for stage st, refill the stage read last time and return st's LDS address.
  int cur = 0, nxt = STAGES - 1;
  auto begin_stage = [&](int st) __attribute__((always_inline)) {
    wait_vmcnt<(STAGES - 2) * T::LOADS>();
    __syncthreads();
    issue(min(st + STAGES - 1, st_end - 1), nxt);
    const char* sp = smem + cur * T::STAGE;
    cur = cur == STAGES - 1 ? 0 : cur + 1;
    nxt = nxt == STAGES - 1 ? 0 : nxt + 1;
    return sp;
  };
  // Two product buffers fit the register file only for up to 4 tiles per wave.
  constexpr bool kOverlap = TM * TN <= 4;
  // One 64-wide group gi of a stage: multiply into pn (scale sn) and meanwhile fold the previous
  // group's product po (scale so) into the accumulators, so that those FMAs overlap this group's
  // MFMAs instead of waiting for them.
  auto group = [&](const char* sp, int gi, f16v (&pn)[TM][TN], float (&sn)[TN],
                   const f16v (&po)[TM][TN], const float (&so)[TN]) __attribute__((always_inline)) {
    h8 bw[TN][4];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const u32x4 raw = *reinterpret_cast<const u32x4*>(sp + (boff[j] ^ (16 * (4 * gi + u))));
        uint32_t h[8];
        i8x4_to_h4(raw.x, h[0], h[1]);
        i8x4_to_h4(raw.y, h[2], h[3]);
        i8x4_to_h4(raw.z, h[4], h[5]);
        i8x4_to_h4(raw.w, h[6], h[7]);
        const u32x4 a = {h[0], h[1], h[2], h[3]};
        const u32x4 b = {h[4], h[5], h[6], h[7]};
        bw[j][2 * u] = __builtin_bit_cast(h8, a);
        bw[j][2 * u + 1] = __builtin_bit_cast(h8, b);
      }
    }
#pragma unroll
    for (int j = 0; j < TN; ++j)
      sn[j] = *reinterpret_cast<const float*>(sp + scoff[j] + gi * T::BN * 8);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      h8 ah[TM], al[TM];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        ah[i] = *reinterpret_cast<const h8*>(sp + (aoff[i] ^ (16 * (8 * gi + t))));
        al[i] = *reinterpret_cast<const h8*>(sp + T::XB + (aoff[i] ^ (16 * (8 * gi + t))));
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          if (t == 0) {
            const f16v zero = {};
            pn[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bw[j][t], zero, 0, 0, 0);
          } else {
            pn[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i], bw[j][t], pn[i][j], 0, 0, 0);
          }
          pn[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], bw[j][t], pn[i][j], 0, 0, 0);
        }
      // a quarter of the previous group's FMAs per K step
      if constexpr (kOverlap) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 4 * t; r < 4 * t + 4; ++r)
              acc[i][j][r] = fmaf(so[j], po[i][j][r], acc[i][j][r]);
      }
    }
  };
  auto fold = [&](const f16v (&po)[TM][TN], const float (&so)[TN]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = fmaf(so[j], po[i][j][r], acc[i][j][r]);
  };
  f16v p0[TM][TN], p1[TM][TN];
  float s0[TN], s1[TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      s0[j] = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) p0[i][j][r] = 0.f;
    }
  if constexpr (!kOverlap) {  // one product buffer: fold each group right after its MFMAs
    for (int st = st_begin; st < st_end; ++st) {
      const char* sp = begin_stage(st);
#pragma unroll
      for (int gi = 0; gi < GPS; ++gi) {
        group(sp, gi, p1, s1, p0, s0);
        fold(p1, s1);
      }
    }
  } else if constexpr (GPS == 2) {  // p1 and p0 alternate within each stage
    for (int st = st_begin; st < st_end; ++st) {
      const char* sp = begin_stage(st);
      group(sp, 0, p1, s1, p0, s0);
      group(sp, 1, p0, s0, p1, s1);
    }
    fold(p0, s0);
  } else {  // p0 and p1 alternate over stage pairs (p0 starts as a zero product)
    int st = st_begin;
    for (; st + 1 < st_end; st += 2) {
      group(begin_stage(st), 0, p1, s1, p0, s0);
      group(begin_stage(st + 1), 0, p0, s0, p1, s1);
    }
    if (st < st_end) {
      group(begin_stage(st), 0, p1, s1, p0, s0);
      fold(p1, s1);
    } else {
      fold(p0, s0);
    }
  }
  // Drain the clamped tail loads before the workgroup's LDS is released.
  wait_vmcnt<0>();

  if (gridDim.z > 1) {  // split-K partial tile: raw sums at the weight row's column
    float* dst = out + static_cast<size_t>(bz) * M * N;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = m0 + (wm * TM + i) * 32 + 8 * (r >> 2) + half * 4 + (r & 3);
        if (m >= M) continue;
        const float rsc = rscale[m];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int c = (wn * TN + j) * 32 + lrow;
          const bool in = swiglu ? feat(c) < F : n0 + c < N;
          if (in) dst[static_cast<size_t>(m) * N + wrow(c)] = acc[i][j][r] * rsc;
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = m0 + (wm * TM + i) * 32 + 8 * (r >> 2) + half * 4 + (r & 3);
      if (m >= M) continue;
      const float rsc = rscale[m];
      if (swiglu) {
#pragma unroll
        for (int jj = 0; jj < HT; ++jj) {
          const int f = f0 + (wn * HT + jj) * 32 + lrow;
          if (f < F)
            out[static_cast<size_t>(m) * F + f] =
                silu_mul(acc[i][jj][r] * rsc, acc[i][jj + HT][r] * rsc);
        }
        continue;
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = n0 + (wn * TN + j) * 32 + lrow;
        if (n >= N) continue;
        const size_t o = static_cast<size_t>(m) * N + n;
        const float v = acc[i][j][r] * rsc;
        out[o] = epi.mode == kEpiResidual ? epi.res[o] + v : v;
      }
    }
  }
}

// ---------------------------------------------------------------- skinny decode kernel
// For 3 <= M <= 64 token rows: one launch, no activation prologue, v_mfma_f32_16x16x32_f16 on
// MT16 stacked 16-row tiles. A workgroup (4 waves) owns BN = 64*TN output columns, all M rows and
// a range of K groups (its split), walked in chunks of KW groups. A wave owns only 16*TN columns,
// so many waves are in flight per CU, which is what hides HBM latency at these sizes:
//  * the wave's weights go from HBM straight into MFMA B registers, double-buffered across
//    chunks; scales ride with them;
//  * the M x (64*KW) activation chunk is split to f16 hi/lo in LDS once per chunk with one power
//    of two per (row, group) from that row's group absmax, so any activation range is safe;
//  * per group, acc += (scale[n, g] * 2^-e[m, g]) * P for the group product P;
//  * lane l: weight row n0 + l%16, the 16 contiguous bytes (l/16)*16.. of each 64-wide group (one
//    dwordx4 per lane per group; a wave instruction covers 16 rows x 64 B);
//  * A operand for step t in {0,1}: x[m = l%16][(l/16)*16 + 8t .. +8] from LDS (hi, lo);
//  * result lane l: column l%16, rows 4*(l/16) .. +3.
// Split-K partials are exchanged with agent-scope atomic stores and loads (coherent across the
// XCDs' L2s), published by a release fence before the workgroup takes its ticket and acquired by
// the last workgroup before it sums them.
typedef float f4v __attribute__((ext_vector_type(4)));

template <int MR, int KW, int TN, int MT16, bool F4>
__global__ __launch_bounds__(kThreads) void skinny16_kernel(
    const float* x, const int8_t* w, const float* s, float* __restrict__ y, float* __restrict__ part, unsigned* __restrict__ tickets, int M, int N,
    int K, int gs, int gps, int splits, int pk) {
  constexpr int BMP = 16 * MT16;                   // MFMA rows: MT16 stacked 16-row tiles
  static_assert(MR <= BMP && (MR == 8 || MR % 16 == 0), "rows loaded per chunk");
  constexpr int BN = 4 * TN * 16;                  // 4 waves x TN tiles of 16 columns
  constexpr int XF4 = MR * KW * 16 / kThreads;     // float4 of an activation chunk per thread
  static_assert(XF4 >= 1, "chunk too small for the staging pattern");
  constexpr int GROUP_HALVES = BMP * LDS_STRIDE;
  __shared__ __attribute__((aligned(16))) _Float16 sxh[2][KW * GROUP_HALVES];
  __shared__ __attribute__((aligned(16))) _Float16 sxl[2][KW * GROUP_HALVES];
  __shared__ __attribute__((aligned(16))) float sxs[2][KW * BMP];
  __shared__ int is_last;

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar address math
  const int lcol = lane & 15, kq = (lane >> 4) * 16;
  const int n0 = blockIdx.x * BN;
  const int gbeg = blockIdx.y * gps;
  const int nch = (min(K / BK, gbeg + gps) - gbeg) / KW;
  const int gpr = K / gs;
  const int gstep = wgroup_step(pk);

  if (MR < BMP) {  // rows MR..15 of both buffers are never loaded: zero them once
    for (int i = tid; i < 2 * KW * (BMP - MR) * LDS_STRIDE; i += kThreads) {
      const int b = i / (KW * (BMP - MR) * LDS_STRIDE), r = i % (KW * (BMP - MR) * LDS_STRIDE);
      const int q = r / ((BMP - MR) * LDS_STRIDE), o = r % ((BMP - MR) * LDS_STRIDE);
      sxh[b][q * GROUP_HALVES + MR * LDS_STRIDE + o] = static_cast<_Float16>(0.f);
      sxl[b][q * GROUP_HALVES + MR * LDS_STRIDE + o] = static_cast<_Float16>(0.f);
    }
    for (int i = tid; i < 2 * KW * (BMP - MR); i += kThreads) {
      const int b = i / (KW * (BMP - MR)), r = i % (KW * (BMP - MR));
      sxs[b][(r / (BMP - MR)) * BMP + MR + r % (BMP - MR)] = 0.f;
    }
  }

  const int8_t* wsrc[TN];
  const float* ssrc[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int ncol = ix::skinny_row(n0, wave, TN, j, lcol, N);
    wsrc[j] = lane_wbase(w, pk, ncol, K, lane) + static_cast<size_t>(gbeg) * gstep;
    ssrc[j] = s + static_cast<size_t>(ncol) * gpr;
  }

  u32x4 wr[2][KW][TN];
  float wsc[2][KW][TN];
  auto wload = [&](int b, int c) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < KW; ++q)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        wr[b][q][j] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(wsrc[j] + (c * KW + q) * gstep));
        if constexpr (!F4) wsc[b][q][j] = ssrc[j][((gbeg + c * KW + q) * BK) / gs];
      }
    if constexpr (F4) {  // group_size 64, KW == 4: the chunk's 4 scales of a row are one float4
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const float4 v = *reinterpret_cast<const float4*>(ssrc[j] + gbeg + c * KW);
        wsc[b][0][j] = v.x;
        wsc[b][1][j] = v.y;
        wsc[b][2][j] = v.z;
        wsc[b][3][j] = v.w;
      }
    }
  };
  float4 xr[XF4];
  auto xload = [&](int c) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < XF4; ++i) {
      const int f = tid + kThreads * i;
      const int row = f / (KW * 16), rem = f % (KW * 16);
      xr[i] = *reinterpret_cast<const float4*>(x + static_cast<size_t>(min(row, M - 1)) * K +
                                               (gbeg + c * KW) * BK + rem * 4);
    }
  };
  auto xstore = [&](int b) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < XF4; ++i) {
      const int f = tid + kThreads * i;
      const int row = f / (KW * 16), rem = f % (KW * 16), q = rem >> 4, part4 = rem & 15;
      const float4 v = row < M ? xr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
      float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
      for (int off = 8; off >= 1; off /= 2) amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
      int e = 0;
      if (amax > 0.f && amax <= 3.402823466e38f) {
        int ex;
        frexpf(amax, &ex);
        e = min(max(14 - ex, -126), 126);
      }
      const float a[4] = {ldexpf(v.x, e), ldexpf(v.y, e), ldexpf(v.z, e), ldexpf(v.w, e)};
      _Float16 h[4], l[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        h[c] = static_cast<_Float16>(a[c]);
        l[c] = static_cast<_Float16>(a[c] - static_cast<float>(h[c]));
      }
      const int o = q * GROUP_HALVES + row * LDS_STRIDE + part4 * 4;
      *reinterpret_cast<uint2*>(&sxh[b][o]) = *reinterpret_cast<const uint2*>(h);
      *reinterpret_cast<uint2*>(&sxl[b][o]) = *reinterpret_cast<const uint2*>(l);
      if (part4 == 0) sxs[b][q * BMP + row] = ldexpf(1.f, -e);
    }
  };

  static_assert(!F4 || KW == 4, "float4 scales cover a 4-group chunk");
  f4v acc[MT16][TN];
#pragma unroll
  for (int i = 0; i < MT16; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f4v{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int b) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < KW; ++q) {
      h8 bw[TN][2];
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        uint32_t hq[8];
        i8x4_to_h4(wr[b][q][j].x, hq[0], hq[1]);
        i8x4_to_h4(wr[b][q][j].y, hq[2], hq[3]);
        i8x4_to_h4(wr[b][q][j].z, hq[4], hq[5]);
        i8x4_to_h4(wr[b][q][j].w, hq[6], hq[7]);
        const u32x4 b0 = {hq[0], hq[1], hq[2], hq[3]};
        const u32x4 b1 = {hq[4], hq[5], hq[6], hq[7]};
        bw[j][0] = __builtin_bit_cast(h8, b0);
        bw[j][1] = __builtin_bit_cast(h8, b1);
      }
#pragma unroll
      for (int i = 0; i < MT16; ++i) {
        const int o = q * GROUP_HALVES + (i * 16 + lcol) * LDS_STRIDE + kq;
        const h8 ah0 = *reinterpret_cast<const h8*>(&sxh[b][o]);
        const h8 al0 = *reinterpret_cast<const h8*>(&sxl[b][o]);
        const h8 ah1 = *reinterpret_cast<const h8*>(&sxh[b][o + 8]);
        const h8 al1 = *reinterpret_cast<const h8*>(&sxl[b][o + 8]);
        const float4 rs =
            *reinterpret_cast<const float4*>(&sxs[b][q * BMP + i * 16 + (lane >> 4) * 4]);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const f4v zero = {0.f, 0.f, 0.f, 0.f};
          f4v p = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah0, bw[j][0], zero, 0, 0, 0);
          p = __builtin_amdgcn_mfma_f32_16x16x32_f16(al0, bw[j][0], p, 0, 0, 0);
          p = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah1, bw[j][1], p, 0, 0, 0);
          p = __builtin_amdgcn_mfma_f32_16x16x32_f16(al1, bw[j][1], p, 0, 0, 0);
          // (scale * partial) * 2^-e: the product scale * 2^-e alone can underflow for tiny rows.
          const float sc = wsc[b][q][j];
          acc[i][j][0] = fmaf(sc * p[0], rs.x, acc[i][j][0]);
          acc[i][j][1] = fmaf(sc * p[1], rs.y, acc[i][j][1]);
          acc[i][j][2] = fmaf(sc * p[2], rs.z, acc[i][j][2]);
          acc[i][j][3] = fmaf(sc * p[3], rs.w, acc[i][j][3]);
        }
      }
    }
  };

  // Chunk c: weights in wr[c & 1], activations in LDS buffer c & 1. The next chunk's activation
  // loads are issued before its weight loads (compiler and scheduling barriers keep that order):
  // vmcnt retires in issue order, so waiting for the activations leaves the weight prefetch in
  // flight. The prefetch and the store of the next buffer are unconditional (past the end they
  // repeat the last chunk into the buffer that is not read again): a load issued on only one
  // branch makes the compiler's wait counts assume the other branch, and the wait for this
  // chunk's data would then also wait for the whole prefetch.
  if (nch > 0) {
    xload(0);
    wload(0, 0);
    xstore(0);
  }
  __syncthreads();
  auto step = [&](auto buf, int c) __attribute__((always_inline)) {
    constexpr int B = decltype(buf)::value;
    const int cn = min(c + 1, nch - 1);
    asm volatile("" ::: "memory");
    xload(cn);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    wload(B ^ 1, cn);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    compute(B);
    __builtin_amdgcn_sched_barrier(0);
    xstore(B ^ 1);
    __syncthreads();
  };
  for (int c = 0; c < nch;) {
    step(std::integral_constant<int, 0>{}, c);
    if (++c >= nch) break;
    step(std::integral_constant<int, 1>{}, c);
    ++c;
  }

  if (splits == 1) {
#pragma unroll
    for (int t = 0; t < MT16; ++t)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = n0 + (wave * TN + j) * 16 + lcol;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = t * 16 + (lane >> 4) * 4 + i;
          if (m < M && n < N) y[static_cast<size_t>(m) * N + n] = acc[t][j][i];
        }
      }
    return;
  }
  float* dst = part + static_cast<size_t>(blockIdx.y) * M * N;
#pragma unroll
  for (int t = 0; t < MT16; ++t)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + (wave * TN + j) * 16 + lcol;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = t * 16 + (lane >> 4) * 4 + i;
        if (m < M && n < N)
          __hip_atomic_store(dst + static_cast<size_t>(m) * N + n, acc[t][j][i],
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  publish_partials();
  __syncthreads();
  if (tid == 0)
    is_last = __hip_atomic_fetch_add(&tickets[blockIdx.x], 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT) == static_cast<unsigned>(splits - 1);
  __syncthreads();
  if (!is_last) return;
  acquire_partials();
  const int ncols = min(BN, N - n0);
  for (int idx = tid; idx < M * ncols; idx += kThreads) {
    const int m = idx / ncols, nn = n0 + idx % ncols;
    const size_t o = static_cast<size_t>(m) * N + nn;
    float v = __hip_atomic_load(part + o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int z = 1; z < splits; ++z)
      v += __hip_atomic_load(part + static_cast<size_t>(z) * M * N + o, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    y[o] = v;
  }
  if (tid == 0)
    __hip_atomic_store(&tickets[blockIdx.x], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- int8-limb decode kernel
// For 1 <= M <= 4*NB token rows on v_mfma_i32_16x16x64_i8, with the int8 weights as the B operand
// exactly as they sit in memory (no conversion at all). Each activation row t is split per 64-wide
// group g into a power of two and four signed 7-bit limbs:
//     round(x * 2^e) = ((a0*128 + a1)*128 + a2)*128 + a3,  |round(x * 2^e)| < 2^27, |aj| <= 64
// where 2^e puts the row's group absmax in [2^25, 2^26): 27 significant bits per element relative
// to its group's absmax. Rows 4t+j of the A operand hold limb j of token t, so one MFMA gives, in
// int32 and exactly, the four limb dot products of up to 4 tokens against 16 output columns over a
// whole group; each lane then combines the four sums of its (token, column) in fp32 and adds
// scale[n, g] * 2^-e * sum. Everything else (chunked double-buffered weight registers, activation
// limbs staged once per workgroup in LDS, fence-free split-K) is as in the f16 skinny kernel.
//  * lane l, weight tile j: row n0 + 16j + l%16, bytes (l/16)*16 .. +16 of each group (B operand);
//  * A operand: row l%16 (token (l%16)/4, limb l%4), the same 16 k positions, from LDS;
//  * result lane l: column l%16, rows 4*(l/16) + i = limbs i of token l/16 (in row block b).
typedef int i32x4v __attribute__((ext_vector_type(4)));
constexpr int kLimbRowBytes = 80;  // 64 limb bytes + 16 padding: conflict-free ds_read_b128

template <int NB, int KW, int TN, bool F4>
__global__ __launch_bounds__(kThreads) void skinny_i8_kernel(
    const float* x, const int8_t* w, const float* s, float* __restrict__ y, float* __restrict__ part, unsigned* __restrict__ tickets, int M, int N,
    int K, int gs, int gps, int splits, int pk) {
  constexpr int MT = 4 * NB;                       // token slots
  constexpr int ROWS = 16 * NB;                    // A rows (4 limbs per token)
  constexpr int BN = 4 * TN * 16;                  // 4 waves x TN tiles of 16 columns
  constexpr int GROUP_BYTES = ROWS * kLimbRowBytes;
  // Activation staging: one thread per (token, group, 4 consecutive k).
  constexpr int XJOBS = MT * KW * 16;
  constexpr int XPT = (XJOBS + kThreads - 1) / kThreads;
  __shared__ __attribute__((aligned(16))) int8_t sa[2][KW * GROUP_BYTES];
  __shared__ __attribute__((aligned(16))) float sx2[2][KW * MT];  // 2^-e per (group, token)
  __shared__ int is_last;

  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar address math
  const int lcol = lane & 15, kq = (lane >> 4) * 16;
  const int n0 = blockIdx.x * BN;
  const int gbeg = blockIdx.y * gps;
  const int nch = (min(K / BK, gbeg + gps) - gbeg) / KW;
  const int gpr = K / gs;
  const int gstep = wgroup_step(pk);

  const int8_t* wsrc[TN];
  const float* ssrc[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int ncol = ix::skinny_row(n0, wave, TN, j, lcol, N);
    wsrc[j] = lane_wbase(w, pk, ncol, K, lane) + static_cast<size_t>(gbeg) * gstep;
    ssrc[j] = s + static_cast<size_t>(ncol) * gpr;
  }

  i32x4v wr[2][KW][TN];
  float wsc[2][KW][TN];
  auto wload = [&](int b, int c) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < KW; ++q)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        wr[b][q][j] = __builtin_nontemporal_load(
            reinterpret_cast<const i32x4v*>(wsrc[j] + (c * KW + q) * gstep));
        if constexpr (!F4) wsc[b][q][j] = ssrc[j][((gbeg + c * KW + q) * BK) / gs];
      }
    if constexpr (F4) {  // group_size 64, KW == 4: the chunk's 4 scales of a row are one float4
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const float4 v = *reinterpret_cast<const float4*>(ssrc[j] + gbeg + c * KW);
        wsc[b][0][j] = v.x;
        wsc[b][1][j] = v.y;
        wsc[b][2][j] = v.z;
        wsc[b][3][j] = v.w;
      }
    }
  };
  float4 xr[XPT];
  auto xload = [&](int c) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int f = min(tid + kThreads * i, XJOBS - 1);
      const int t = f / (KW * 16), rem = f % (KW * 16);
      xr[i] = *reinterpret_cast<const float4*>(x + static_cast<size_t>(min(t, M - 1)) * K +
                                               (gbeg + c * KW) * BK + rem * 4);
    }
  };
  auto xstore = [&](int b) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const int f = tid + kThreads * i;
      const bool job = f < XJOBS;
      const int fc = min(f, XJOBS - 1);
      const int t = fc / (KW * 16), rem = fc % (KW * 16), q = rem >> 4, part4 = rem & 15;
      const float4 v = (job && t < M) ? xr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
      float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
      for (int off = 8; off >= 1; off /= 2) amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
      int e = 0;
      if (amax > 0.f && amax <= 3.402823466e38f) {
        int ex;
        frexpf(amax, &ex);
        e = min(max(26 - ex, -126), 126);
      }
      const float xf[4] = {v.x, v.y, v.z, v.w};
      uint32_t limb[4] = {0u, 0u, 0u, 0u};  // limb j of the 4 elements, one byte each
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        int X = static_cast<int>(rintf(ldexpf(xf[c], e)));
#pragma unroll
        for (int j = 3; j >= 1; --j) {
          const int a = ((X + 64) & 127) - 64;
          limb[j] |= (static_cast<uint32_t>(a) & 0xffu) << (8 * c);
          X = (X - a) >> 7;
        }
        limb[0] |= (static_cast<uint32_t>(X) & 0xffu) << (8 * c);
      }
      if (job) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *reinterpret_cast<uint32_t*>(&sa[b][q * GROUP_BYTES + (4 * t + j) * kLimbRowBytes +
                                            part4 * 4]) = limb[j];
        if (part4 == 0) sx2[b][q * MT + t] = ldexpf(1.f, -e);
      }
    }
  };

  static_assert(!F4 || KW == 4, "float4 scales cover a 4-group chunk");
  float acc[NB][TN];
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[b][j] = 0.f;
  auto compute = [&](int bb) __attribute__((always_inline)) {
#pragma unroll
    for (int q = 0; q < KW; ++q) {
#pragma unroll
      for (int rb = 0; rb < NB; ++rb) {
        const i32x4v a = *reinterpret_cast<const i32x4v*>(
            &sa[bb][q * GROUP_BYTES + (rb * 16 + lcol) * kLimbRowBytes + kq]);
        const float r2 = sx2[bb][q * MT + rb * 4 + (lane >> 4)];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const i32x4v zero = {0, 0, 0, 0};
          const i32x4v d = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, wr[bb][q][j], zero, 0, 0, 0);
          // ((c0*128 + c1)*128 + c2)*128 + c3 = sum of round(x * 2^e) * q; times scale * 2^-e
          float v = static_cast<float>(d[0]);
          v = fmaf(v, 128.f, static_cast<float>(d[1]));
          v = fmaf(v, 128.f, static_cast<float>(d[2]));
          v = fmaf(v, 128.f, static_cast<float>(d[3]));
          // scale * v is the partial for activations normalised to [2^25, 2^26): in range for any
          // finite weight scale. Folding 2^-e into the scale first would underflow for tiny rows.
          acc[rb][j] = fmaf(wsc[bb][q][j] * v, r2, acc[rb][j]);
        }
      }
    }
  };

  // Zero both LDS buffers once: token slots >= M stay zero.
  for (int i = tid * 4; i < 2 * KW * GROUP_BYTES; i += kThreads * 4)
    *reinterpret_cast<uint32_t*>(&sa[0][0] + i) = 0u;
  __syncthreads();
  if (nch > 0) {
    xload(0);
    wload(0, 0);
    xstore(0);
  }
  __syncthreads();
  // Branch-free steps, as in the f16 skinny kernel: the prefetch and the store of the next
  // buffer are unconditional (past the end they repeat the last chunk into the buffer that is
  // not read again), so the compiler's wait counts never assume a branch without the prefetch.
  auto step = [&](auto buf, int c) __attribute__((always_inline)) {
    constexpr int B = decltype(buf)::value;
    const int cn = min(c + 1, nch - 1);
    asm volatile("" ::: "memory");
    xload(cn);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    wload(B ^ 1, cn);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    compute(B);
    __builtin_amdgcn_sched_barrier(0);
    xstore(B ^ 1);
    __syncthreads();
  };
  for (int c = 0; c < nch;) {
    step(std::integral_constant<int, 0>{}, c);
    if (++c >= nch) break;
    step(std::integral_constant<int, 1>{}, c);
    ++c;
  }

  // Lane l holds token 4*rb + l/16 of column (tile) + l%16.
  if (splits == 1) {
#pragma unroll
    for (int rb = 0; rb < NB; ++rb)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int m = rb * 4 + (lane >> 4), n = n0 + (wave * TN + j) * 16 + lcol;
        if (m < M && n < N) y[static_cast<size_t>(m) * N + n] = acc[rb][j];
      }
    return;
  }
  float* dst = part + static_cast<size_t>(blockIdx.y) * M * N;
#pragma unroll
  for (int rb = 0; rb < NB; ++rb)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int m = rb * 4 + (lane >> 4), n = n0 + (wave * TN + j) * 16 + lcol;
      if (m < M && n < N)
        __hip_atomic_store(dst + static_cast<size_t>(m) * N + n, acc[rb][j], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
  publish_partials();
  __syncthreads();
  if (tid == 0)
    is_last = __hip_atomic_fetch_add(&tickets[blockIdx.x], 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT) == static_cast<unsigned>(splits - 1);
  __syncthreads();
  if (!is_last) return;
  acquire_partials();
  const int ncols = min(BN, N - n0);
  for (int idx = tid; idx < M * ncols; idx += kThreads) {
    const int m = idx / ncols, nn = n0 + idx % ncols;
    const size_t o = static_cast<size_t>(m) * N + nn;
    float v = __hip_atomic_load(part + o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int z = 1; z < splits; ++z)
      v += __hip_atomic_load(part + static_cast<size_t>(z) * M * N + o, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    y[o] = v;
  }
  if (tid == 0)
    __hip_atomic_store(&tickets[blockIdx.x], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- small-batch decode tile kernel
// For 5 <= M <= 64 token rows. Two launches:
//  * pack_x_kernel splits each token row into f16 hi/lo halves with one power of two per row (the
//    same split as split_x_kernel) and writes them in MFMA fragment order, so that a wave fetches
//    the A operand of one 64-wide group for 16 rows with four fully coalesced dwordx4 loads:
//        xp[g][rt][u][lane] (16 bytes each), u = 2*t + (0 hi | 1 lo), t = K half-step,
//        lane l holds row 16*rt + l%16, k = 64*g + (l/16)*16 + 8*t .. +8.
//    Rows M .. 16*RT-1 are written as zeros.
//  * tile_kernel: a workgroup of W waves owns 16*T output columns and a range of K groups; wave w
//    takes groups w, w + W, w + 2W, ... of that range, so the W waves of a workgroup together
//    stream the weight tile front to back. Per group a lane loads, for each of its T column tiles,
//    the 16 contiguous weight bytes (l/16)*16 .. of row n0 + 16j + l%16 straight into B registers,
//    plus the tile's scale and the RT*4 A fragments; the next group's loads are issued before the
//    current group is multiplied (register double buffer). No barrier until the end: the W
//    per-wave accumulators are summed in LDS in wave order (deterministic), multiplied by the
//    row's 2^-e and written (or, with K split over gridDim.y, passed through the split-K tickets
//    as in the skinny kernels).
// Per group and column tile: P = sum of the hi and lo MFMAs over both half-steps (from zero),
// acc += scale[n, g] * P. Result lane l: column l%16, rows 16*rt + 4*(l/16) .. +3.
//
// With NORM the packed row is rmsnorm(x + res) * nw instead (the reference's add + RMSNorm ahead
// of a projection, rmsnorm_kernel.cu): x + res is written back to x (res may be null), the row
// stays in registers (K <= kSplitThreads * 4 * kSplitV) and one workgroup owns the row, so the
// write-back is in place.
template <bool NORM>
__global__ __launch_bounds__(kSplitThreads) void pack_x_kernel(const float* x,
                                                             uint2* __restrict__ xp,
                                                             float* __restrict__ rscale, int M,
                                                             int K, int RT, NormArgs na) {
  __shared__ float red[kSplitThreads / kWave];
  const int m = blockIdx.x;
  const int rt = m >> 4;
  const bool live = m < M;
  const float* xr = x + static_cast<size_t>(min(m, M - 1)) * K;
  float4 v[kSplitV];
  int e;
  if constexpr (NORM) {
    const int tid = threadIdx.x;
    const size_t row = static_cast<size_t>(min(m, M - 1)) * K;
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kSplitV; ++i) {
      const int k = (tid + i * kSplitThreads) * 4;
      const bool in = live && k < K;
      v[i] = in ? *reinterpret_cast<const float4*>(xr + k) : make_float4(0.f, 0.f, 0.f, 0.f);
      if (na.res && in) {
        const float4 r = *reinterpret_cast<const float4*>(na.res + row + k);
        v[i] = make_float4(v[i].x + r.x, v[i].y + r.y, v[i].z + r.z, v[i].w + r.w);
      }
      ss = fmaf(v[i].x, v[i].x, ss);
      ss = fmaf(v[i].y, v[i].y, ss);
      ss = fmaf(v[i].z, v[i].z, ss);
      ss = fmaf(v[i].w, v[i].w, ss);
    }
#pragma unroll
    for (int off = 32; off >= 1; off /= 2) ss += __shfl_xor(ss, off, kWave);
    if ((tid & (kWave - 1)) == 0) red[tid >> 6] = ss;
    __syncthreads();
    float total = red[0];
#pragma unroll
    for (int w = 1; w < kSplitThreads / kWave; ++w) total += red[w];
    const float scale = rsqrtf(total / static_cast<float>(K) + na.eps);
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < kSplitV; ++i) {
      const int k = (tid + i * kSplitThreads) * 4;
      if (live && k < K) {
        if (na.res) *reinterpret_cast<float4*>(na.x + row + k) = v[i];
        const float4 g = *reinterpret_cast<const float4*>(na.w + k);
        v[i] = make_float4(scale * v[i].x * g.x, scale * v[i].y * g.y, scale * v[i].z * g.z,
                           scale * v[i].w * g.w);
      }
      amax = fmaxf(amax, absmax4(v[i]));
    }
#pragma unroll
    for (int off = 32; off >= 1; off /= 2) amax = fmaxf(amax, __shfl_xor(amax, off, kWave));
    __syncthreads();  // every wave has read the sums before red is reused
    if ((tid & (kWave - 1)) == 0) red[tid >> 6] = amax;
    __syncthreads();
    amax = red[0];
#pragma unroll
    for (int w = 1; w < kSplitThreads / kWave; ++w) amax = fmaxf(amax, red[w]);
    e = row_exponent(amax);
  } else {
    e = load_row_exponent(xr, K, live, v, red);
  }
  if (live && threadIdx.x == 0) rscale[m] = ldexpf(1.f, -e);
  for_row_chunks(xr, K, live, v, [&](int k, float4 c) {
    _Float16 h[4], l[4];
    split4(c, e, h, l);
    const int g = k >> 6, kk = k & 63, t = (kk >> 3) & 1, half = (kk >> 2) & 1;
    const int lane = (kk >> 4) * 16 + (m & 15);
    // uint2 index: 16-byte fragment (g, rt, u, lane) holds two uint2; `half` picks one.
    const size_t frag = ((static_cast<size_t>(g) * RT + rt) * 4 + 2 * t) * kWave + lane;
    xp[frag * 2 + half] = *reinterpret_cast<const uint2*>(h);
    xp[(frag + kWave) * 2 + half] = *reinterpret_cast<const uint2*>(l);
  });
}

template <int RT, int T, int W>
__global__ __launch_bounds__(W * kWave) void tile_kernel(
    const u32x4* xp, const float* __restrict__ rscale, const int8_t* w, const float* s,
    float* __restrict__ y, float* __restrict__ part,
    unsigned* __restrict__ tickets, int M, int N, int K, int gs, int gps, int splits, int pk) {
  constexpr int OUTS = RT * T * 4 * kWave;  // accumulator floats per wave
  constexpr int NT = W * kWave;
  constexpr int SROWS = 16 * T;             // weight rows (output columns) of the workgroup
  constexpr int LDSF = (W > 1 ? W * OUTS : 0) > SROWS * (kTileScaleGroups + 1)
                           ? W * OUTS : SROWS * (kTileScaleGroups + 1);
  static_assert(LDSF * 4 <= 64 * 1024, "tile_kernel LDS above 64 KiB");
  // Scale stage [SROWS][gps] during the main loop, then the cross-wave reduction buffer.
  __shared__ float lds[LDSF];
  __shared__ int is_last;

  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lcol = lane & 15;
  const int n0 = blockIdx.x * (16 * T);
  const int G = K / BK, gpr = K / gs;
  const int gsplit = blockIdx.y * gps;              // first group of this split
  const int gcount = min(G, gsplit + gps) - gsplit; // groups in this split (<= kTileScaleGroups)
  const int nst = wave < gcount ? (gcount - wave + W - 1) / W : 0;
  const int sstride = gcount + 1;  // padded: the 16 lanes of a column read distinct banks

  // Stage the split's scales of the workgroup's rows in LDS: row-contiguous, coalesced loads.
  // Per-lane loads in the MFMA layout would touch 16 rows per instruction, once per group.
  for (int idx = tid; idx < SROWS * gcount; idx += NT) {
    const int r = idx / gcount, gi = idx - r * gcount;
    const int n = min(n0 + r, N - 1);
    lds[r * sstride + gi] = s[static_cast<size_t>(n) * gpr + ((gsplit + gi) * BK) / gs];
  }

  const int8_t* wrow[T];
#pragma unroll
  for (int j = 0; j < T; ++j)
    wrow[j] = lane_wbase(w, pk, ix::tile_row(n0, j, lcol, N), K, lane);
  const int gstep = wgroup_step(pk);
  const u32x4* xlane = xp + lane;

  // Wave w takes groups w, w + W, ... of the split: the W waves of a workgroup read neighbouring
  // 64-byte pieces of the same rows at about the same time, which streams best from HBM.
  u32x4 bq[2][T];
  u32x4 af[2][RT][4];
  bool live_b[2];
  int gi_b[2];
  // Step i >= nst (the padding to an even count) re-reads the last group with scale 0.
  auto load = [&](int b, int i) __attribute__((always_inline)) {
    const int gi = wave + min(i, nst - 1) * W;
    const int g = gsplit + gi;
#pragma unroll
    for (int j = 0; j < T; ++j)
      bq[b][j] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(wrow[j] + static_cast<size_t>(g) * gstep));
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int u = 0; u < 4; ++u)
        af[b][r][u] = xlane[((static_cast<size_t>(g) * RT + r) * 4 + u) * kWave];
    live_b[b] = i < nst;
    gi_b[b] = gi;
  };

  f4v acc[RT][T];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int j = 0; j < T; ++j) acc[r][j] = f4v{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int b) __attribute__((always_inline)) {
    h8 bw[T][2];
    float sc[T];
#pragma unroll
    for (int j = 0; j < T; ++j) {
      uint32_t hq[8];
      i8x4_to_h4(bq[b][j].x, hq[0], hq[1]);
      i8x4_to_h4(bq[b][j].y, hq[2], hq[3]);
      i8x4_to_h4(bq[b][j].z, hq[4], hq[5]);
      i8x4_to_h4(bq[b][j].w, hq[6], hq[7]);
      const u32x4 b0 = {hq[0], hq[1], hq[2], hq[3]};
      const u32x4 b1 = {hq[4], hq[5], hq[6], hq[7]};
      bw[j][0] = __builtin_bit_cast(h8, b0);
      bw[j][1] = __builtin_bit_cast(h8, b1);
      const float v = lds[(16 * j + lcol) * sstride + gi_b[b]];
      sc[j] = live_b[b] ? v : 0.f;
    }
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int j = 0; j < T; ++j) {
        const f4v zero = {0.f, 0.f, 0.f, 0.f};
        f4v p = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, af[b][r][0]),
                                                       bw[j][0], zero, 0, 0, 0);
        p = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, af[b][r][1]), bw[j][0],
                                                   p, 0, 0, 0);
        p = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, af[b][r][2]), bw[j][1],
                                                   p, 0, 0, 0);
        p = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, af[b][r][3]), bw[j][1],
                                                   p, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[r][j][i] = fmaf(sc[j], p[i], acc[r][j][i]);
      }
  };

  // Register double buffer, branch-free: the step count is padded to even and every load is
  // issued unconditionally. A load issued on only one branch makes the compiler's wait counts
  // assume the other branch, and the wait for this step's data would then also wait for most of
  // the prefetch. The streamed pointers are not __restrict__, so the compiler barriers pin the
  // loads to their step. The scale stage was written before the first weight loads, so the
  // barrier's wait for it does not wait for them.
  if (nst > 0) load(0, 0);
  __syncthreads();
  for (int i = 0; i < nst; i += 2) {
    asm volatile("" ::: "memory");
    load(1, i + 1);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    compute(0);
    asm volatile("" ::: "memory");
    load(0, i + 2);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    compute(1);
  }
  __syncthreads();  // the scale stage is reused below

  // Sum the W waves' accumulators in wave order; output o = ((r*T + j)*4 + i)*64 + lane.
  float out[(OUTS + NT - 1) / NT];
  if constexpr (W > 1) {
    float* red = lds;
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int j = 0; j < T; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave * OUTS + ((r * T + j) * 4 + i) * kWave + lane] = acc[r][j][i];
    __syncthreads();
#pragma unroll
    for (int q = 0; q < (OUTS + NT - 1) / NT; ++q) {
      const int o = tid + q * NT;
      float v = 0.f;
      if (o < OUTS)
        for (int z = 0; z < W; ++z) v += lds[z * OUTS + o];
      out[q] = v;
    }
  } else {
#pragma unroll
    for (int r = 0; r < RT; ++r)
#pragma unroll
      for (int j = 0; j < T; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) out[(r * T + j) * 4 + i] = acc[r][j][i];
  }
  auto coords = [&](int q, int& m, int& n) __attribute__((always_inline)) {
    const int o = W > 1 ? tid + q * NT : q * kWave + lane;
    const int ln = o & (kWave - 1), ri = o / kWave;  // ri = (r*T + j)*4 + i
    const int i = ri & 3, j = (ri >> 2) % T, r = (ri >> 2) / T;
    m = 16 * r + 4 * (ln >> 4) + i;
    n = n0 + 16 * j + (ln & 15);
    return o < OUTS;
  };
  constexpr int NQ = (OUTS + NT - 1) / NT;
  if (splits == 1) {
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      int m, n;
      if (coords(q, m, n) && m < M && n < N)
        y[static_cast<size_t>(m) * N + n] = out[q] * rscale[m];
    }
    return;
  }
  float* dst = part + static_cast<size_t>(blockIdx.y) * M * N;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    int m, n;
    if (coords(q, m, n) && m < M && n < N)
      __hip_atomic_store(dst + static_cast<size_t>(m) * N + n, out[q] * rscale[m],
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // The last workgroup of the column block sums the splits in order.
  publish_partials();
  __syncthreads();
  if (tid == 0)
    is_last = __hip_atomic_fetch_add(&tickets[blockIdx.x], 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT) == static_cast<unsigned>(splits - 1);
  __syncthreads();
  if (!is_last) return;
  acquire_partials();
  const int ncols = min(16 * T, N - n0);
  for (int idx = tid; idx < M * ncols; idx += NT) {
    const int m = idx / ncols, nn = n0 + idx % ncols;
    const size_t o = static_cast<size_t>(m) * N + nn;
    float v = __hip_atomic_load(part + o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int z = 1; z < splits; ++z)
      v += __hip_atomic_load(part + static_cast<size_t>(z) * M * N + o, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
    y[o] = v;
  }
  if (tid == 0)
    __hip_atomic_store(&tickets[blockIdx.x], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- decode GEMM (9..64 rows)
// A workgroup of W waves owns 16*T*W output columns and a range of K groups (its split); each
// wave owns 16*T of the columns for all 16*RT token rows. Per 64-wide group:
//  * the activation fragments of the group (pack_x_kernel's MFMA-ready layout, RT*4 KiB) arrive
//    in an S-stage LDS ring by global -> LDS DMA, once per workgroup, and every wave reads them
//    from there (the tile kernel loads them per wave from L2, 4x the weight bytes);
//  * the wave's weights (16 bytes per lane and column tile, v_mfma_f32_16x16x32_f16 B layout) go
//    straight into a D-deep register ring. Under full load the memory latency is several
//    microseconds, and streaming HBM at full rate needs ~128 KiB in flight per CU:
//    D = 8 groups x 8 waves x 2 tiles x 1 KiB;
//  * the split's scales are staged in LDS once, up front, with row-contiguous loads.
// The DMA is issued from inline asm. Each thread issues the same loads per group: the DMA and
// then the weights of the group D-1 ahead (one distance for both: a wait counter drains in order,
// so waiting for a DMA issued closer than the weights would also drain weights meant to stay in
// flight). It waits until the group's DMA and weights have landed, and a barrier publishes the
// stage and frees the one refilled next. Groups past the split re-read its last group with scale
// 0, so every step issues its loads unconditionally.
template <int RT, int T, int W, int D>
__global__ __launch_bounds__(W * kWave) void dgemm_kernel(
    const u32x4* xp, const float* __restrict__ rscale, const int8_t* w, const float* s,
    float* out, int M, int N, int K, int gs, int gps, Epi epi, int pk) {
  constexpr int XSTAGE = RT * 4 * kWave * 16;          // bytes of one group's fragments
  constexpr int NCH = XSTAGE / (kWave * 16);           // 1 KiB chunks of a group's fragments
  constexpr int LXD = (NCH + W - 1) / W;               // DMA instructions per thread per group
  static_assert(T % 2 == 0, "SwiGLU pairs tile j with tile j + T/2");
  constexpr int LOADS = LXD + T;                       // loads per thread per group
  constexpr int WAIT = (D - 2) * LOADS;                // see the step order below
  static_assert(D >= 2 && WAIT < 64, "ring depth");
  constexpr int HT = T / 2;
  constexpr int COLS = 16 * T * W;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lcol = lane & 15;
  const int G = K / BK, gpr = K / gs;
  const int gsplit = blockIdx.y * gps;
  const int gcount = min(G, gsplit + gps) - gsplit;
  const int sstride = gcount + 1;                      // padded: no bank conflicts across lcol
  const bool swiglu = epi.mode == kEpiSwiglu;
  const int F = N / 2;
  const int n0 = blockIdx.x * COLS, f0 = blockIdx.x * (COLS / 2);
  // Weight row of workgroup column c = (wv * T + j) * 16 + l (SwiGLU: tiles j < T/2 hold the gate
  // rows of the wave's features, tiles j >= T/2 the matching up rows).
  auto wrow = [&](int c) __attribute__((always_inline)) {
    return ix::dgemm_row(c, blockIdx.x, T, W, N, swiglu);
  };
  float* sscale = reinterpret_cast<float*>(smem + D * XSTAGE);
  for (int idx = tid; idx < COLS * gcount; idx += W * kWave) {
    const int c = idx / gcount, gi = idx - c * gcount;
    sscale[c * sstride + gi] = s[static_cast<size_t>(wrow(c)) * gpr + ((gsplit + gi) * BK) / gs];
  }
  const int8_t* wr[T];
#pragma unroll
  for (int j = 0; j < T; ++j)
    wr[j] = lane_wbase(w, pk, wrow((wave * T + j) * 16 + lcol), K, lane);
  const int gstep = wgroup_step(pk);
  const float* scol[T];
#pragma unroll
  for (int j = 0; j < T; ++j) scol[j] = sscale + ((wave * T + j) * 16 + lcol) * sstride;

  const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem));
  const int nsteps = gcount;
  auto gclamp = [&](int i) { return gsplit + min(i, nsteps - 1); };
  auto dma_x = [&](int i, int slot) __attribute__((always_inline)) {
    const char* src = reinterpret_cast<const char*>(xp) + static_cast<size_t>(gclamp(i)) * XSTAGE;
    // Every wave issues LXD copies; when the chunks do not divide evenly, the surplus ones copy
    // a chunk again (same bytes to the same place), so all waves count the same loads.
#pragma unroll
    for (int q = 0; q < LXD; ++q) {
      const uint32_t off = static_cast<uint32_t>(((q * W + wave) % NCH) * kWave * 16);
      dma16(src, off + lane * 16u, lds0 + slot * XSTAGE + off);
    }
  };
  // Weight loads from inline asm too: the compiler does not count them, so it inserts no wait
  // of its own; tie() after the wait below keeps every use of a ring slot behind that wait.
  u32x4 wq[D][T];
  auto load_w = [&](int i, int slot) __attribute__((always_inline)) {
    const int g = gclamp(i);
#pragma unroll
    for (int j = 0; j < T; ++j)
      asm volatile("global_load_dwordx4 %0, %1, off nt"
                   : "=v"(wq[slot][j])
                   : "v"(wr[j] + static_cast<size_t>(g) * gstep)
                   : "memory");
  };
  auto tie = [&](int slot) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < T; ++j) asm volatile("" : "+v"(wq[slot][j]));
  };

  f4v acc[RT][T];
#pragma unroll
  for (int r = 0; r < RT; ++r)
#pragma unroll
    for (int j = 0; j < T; ++j) acc[r][j] = f4v{0.f, 0.f, 0.f, 0.f};

  // Prologue: DMA and weights for groups 0 .. D-2 (the scale stage's loads were consumed by its
  // LDS writes above, so they are not outstanding).
#pragma unroll
  for (int p = 0; p < D - 1; ++p) {
    dma_x(p, p);
    load_w(p, p);
  }
  const int nloop = (nsteps + D - 1) / D * D;
  for (int i0 = 0; i0 < nloop; i0 += D) {
#pragma unroll
    for (int b = 0; b < D; ++b) {
      const int i = i0 + b;
      wait_vmcnt<WAIT>();  // group i's DMA and weights (issued D-1 groups ago) have landed
      tie(b);
      __syncthreads();  // publishes stage i (and, the first time, the scale stage)
      asm volatile("" ::: "memory");
      dma_x(i + D - 1, (b + D - 1) % D);
      load_w(i + D - 1, (b + D - 1) % D);
      asm volatile("" ::: "memory");
      const char* xs = smem + b * XSTAGE;
      const bool live = i < nsteps;
      h8 bw[T][2];
      float sc[T];
#pragma unroll
      for (int j = 0; j < T; ++j) {
        uint32_t hq[8];
        i8x4_to_h4(wq[b][j].x, hq[0], hq[1]);
        i8x4_to_h4(wq[b][j].y, hq[2], hq[3]);
        i8x4_to_h4(wq[b][j].z, hq[4], hq[5]);
        i8x4_to_h4(wq[b][j].w, hq[6], hq[7]);
        const u32x4 b0 = {hq[0], hq[1], hq[2], hq[3]};
        const u32x4 b1 = {hq[4], hq[5], hq[6], hq[7]};
        bw[j][0] = __builtin_bit_cast(h8, b0);
        bw[j][1] = __builtin_bit_cast(h8, b1);
        sc[j] = live ? scol[j][min(i, nsteps - 1)] : 0.f;
      }
#pragma unroll
      for (int r = 0; r < RT; ++r) {
        // one row tile's fragments at a time (hoisting all of them spills at RT >= 3)
        if (RT >= 3) __builtin_amdgcn_sched_barrier(0);
        h8 a[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
          a[u] = *reinterpret_cast<const h8*>(xs + ((r * 4 + u) * kWave + lane) * 16);
#pragma unroll
        for (int j = 0; j < T; ++j) {
          const f4v zero = {0.f, 0.f, 0.f, 0.f};
          f4v pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[0], bw[j][0], zero, 0, 0, 0);
          pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[1], bw[j][0], pr, 0, 0, 0);
          pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[2], bw[j][1], pr, 0, 0, 0);
          pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[3], bw[j][1], pr, 0, 0, 0);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[r][j][e] = fmaf(sc[j], pr[e], acc[r][j][e]);
        }
      }
    }
  }
  wait_vmcnt<0>();  // the clamped tail loads land before the workgroup ends

  // Output: acc[r][j][e] is row 16 r + 4 (lane / 16) + e, column lcol of tile j.
  const bool partial = gridDim.y > 1;
  float* dst = out + (partial ? static_cast<size_t>(blockIdx.y) * M * N : 0);
#pragma unroll
  for (int r = 0; r < RT; ++r) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = 16 * r + 4 * (lane >> 4) + e;
      if (m >= M) continue;
      const float rsc = rscale[m];
      if (swiglu) {
#pragma unroll
        for (int j = 0; j < HT; ++j) {
          const int f = f0 + (wave * HT + j) * 16 + lcol;
          if (f >= F) continue;
          const float g = acc[r][j][e] * rsc, u = acc[r][j + HT][e] * rsc;
          if (partial) {
            dst[static_cast<size_t>(m) * N + f] = g;
            dst[static_cast<size_t>(m) * N + F + f] = u;
          } else {
            dst[static_cast<size_t>(m) * F + f] = silu_mul(g, u);
          }
        }
        continue;
      }
#pragma unroll
      for (int j = 0; j < T; ++j) {
        const int n = n0 + (wave * T + j) * 16 + lcol;
        if (n >= N) continue;
        const size_t o = static_cast<size_t>(m) * N + n;
        const float v = acc[r][j][e] * rsc;
        dst[o] = !partial && epi.mode == kEpiResidual ? epi.res[o] + v : v;
      }
    }
  }
}

// Sum split-K partials in split order, y[i] = sum_z part[z][i], then apply the epilogue:
// residual: y[i] = res[i] + sum; SwiGLU (part holds M rows of N = 2F): y[m][f] =
// silu(gate sum) * (up sum).
__global__ __launch_bounds__(kThreads) void splitk_reduce_kernel(const float* __restrict__ part,
                                                                float* y, int M, int N,
                                                                int splits, Epi epi) {
  const size_t mn = static_cast<size_t>(M) * N;
  const bool swiglu = epi.mode == kEpiSwiglu;
  const int F = N / 2;
  const size_t count = swiglu ? static_cast<size_t>(M) * F : mn;
  for (size_t i = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x; i < count;
       i += static_cast<size_t>(gridDim.x) * kThreads) {
    if (swiglu) {
      const size_t g = (i / F) * N + i % F;
      float a = part[g], b = part[g + F];
      for (int z = 1; z < splits; ++z) {
        a += part[z * mn + g];
        b += part[z * mn + g + F];
      }
      y[i] = silu_mul(a, b);
      continue;
    }
    float v = part[i];
    for (int z = 1; z < splits; ++z) v += part[static_cast<size_t>(z) * mn + i];
    y[i] = epi.mode == kEpiResidual ? epi.res[i] + v : v;
  }
}

// Epilogue of the paths without a fused one: y = epilogue(t) for the finished product t [M][N].
__global__ __launch_bounds__(kThreads) void epilogue_kernel(const float* __restrict__ t, float* y,
                                                           int M, int N, Epi epi) {
  const bool swiglu = epi.mode == kEpiSwiglu;
  const int F = N / 2;
  const size_t count = swiglu ? static_cast<size_t>(M) * F : static_cast<size_t>(M) * N;
  for (size_t i = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x; i < count;
       i += static_cast<size_t>(gridDim.x) * kThreads) {
    if (swiglu) {
      const size_t g = (i / F) * N + i % F;
      y[i] = silu_mul(t[g], t[g + F]);
    } else {
      y[i] = epi.res[i] + t[i];
    }
  }
}

size_t align256(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

Plan make_plan(int M, int N, int K) { return make_plan_for(M, N, K, cu_count()); }

template <int WM, int WN, int TM, int TN, int STAGES, int GPS = 1>
hipError_t launch_gemm(const _Float16* xh, const _Float16* xl, const float* rsc,
                            const int8_t* w, const float* s, float* out, int M, int N, int K,
                            int gs, const Plan& p, hipStream_t st, Epi epi, int pk) {
  using T = PTile<WM, WN, TM, TN, STAGES, GPS>;
  auto kern = gemm_kernel<WM, WN, TM, TN, STAGES, GPS>;
  static std::atomic<uint64_t> done{0};  // LDS above 64 KiB needs the opt-in attribute
  hipError_t e = ensure_dynamic_lds(reinterpret_cast<const void*>(kern), T::LDS_BYTES, done);
  if (e != hipSuccess) return e;
  // SwiGLU: a workgroup owns BN/2 features (their gate and up rows)
  const int cols = epi.mode == kEpiSwiglu ? (N / 2 + T::BN / 2 - 1) / (T::BN / 2)
                                          : (N + T::BN - 1) / T::BN;
  const dim3 grid(cols, (M + T::BM - 1) / T::BM, p.splits);
  hipLaunchKernelGGL(kern, grid, dim3(T::NT), T::LDS_BYTES, st, xh, xl, rsc, w, s, out, M, N, K,
                     gs, p.groups_per_split, epi, pk);
  return hipGetLastError();
}

template <int MR, int KW, int TN = 1, int MT16 = 1>
hipError_t launch_skinny16(const float* x, const int8_t* w, const float* s, float* y, float* part,
                           unsigned* tickets, int M, int N, int K, int gs, const Plan& p,
                           hipStream_t st, int pk) {
  const dim3 grid((N + 64 * TN - 1) / (64 * TN), p.splits);
  // float4 scale loads need 4-group chunks at 16-byte aligned addresses
  const bool f4 = KW == 4 && gs == BK && (K / BK) % 4 == 0 &&
                  (reinterpret_cast<uintptr_t>(s) & 15) == 0;
  if (f4)
    hipLaunchKernelGGL((skinny16_kernel<MR, KW, TN, MT16, KW == 4>), grid, dim3(kThreads), 0, st,
                       x, w, s, y, part, tickets, M, N, K, gs, p.groups_per_split, p.splits, pk);
  else
    hipLaunchKernelGGL((skinny16_kernel<MR, KW, TN, MT16, false>), grid, dim3(kThreads), 0, st, x,
                       w, s, y, part, tickets, M, N, K, gs, p.groups_per_split, p.splits, pk);
  return hipGetLastError();
}

template <int NB, int KW, int TN>
hipError_t launch_skinny_i8(const float* x, const int8_t* w, const float* s, float* y, float* part,
                            unsigned* tickets, int M, int N, int K, int gs, const Plan& p,
                            hipStream_t st, int pk) {
  const dim3 grid((N + 64 * TN - 1) / (64 * TN), p.splits);
  const bool f4 = KW == 4 && gs == BK && (K / BK) % 4 == 0 &&
                  (reinterpret_cast<uintptr_t>(s) & 15) == 0;
  if (f4)
    hipLaunchKernelGGL((skinny_i8_kernel<NB, KW, TN, KW == 4>), grid, dim3(kThreads), 0, st, x,
                       w, s, y, part, tickets, M, N, K, gs, p.groups_per_split, p.splits, pk);
  else
    hipLaunchKernelGGL((skinny_i8_kernel<NB, KW, TN, false>), grid, dim3(kThreads), 0, st, x, w,
                       s, y, part, tickets, M, N, K, gs, p.groups_per_split, p.splits, pk);
  return hipGetLastError();
}

template <int RT>
hipError_t launch_dgemm(const float* x, const int8_t* w, const float* s, float* y, void* ws, int M,
                        int N, int K, int gs, const Plan& p, hipStream_t st, Epi epi,
                        const NormArgs* na, int pk) {
  char* base = static_cast<char*>(ws) + kTicketBytes;
  u32x4* xp = reinterpret_cast<u32x4*>(base);
  base += align256(static_cast<size_t>(K / BK) * RT * 4 * kWave * sizeof(u32x4));
  float* rsc = reinterpret_cast<float*>(base);
  base += align256(static_cast<size_t>(16 * RT) * sizeof(float));
  float* part = reinterpret_cast<float*>(base);
  if (na)
    hipLaunchKernelGGL(pack_x_kernel<true>, dim3(16 * RT), dim3(kSplitThreads), 0, st, x,
                       reinterpret_cast<uint2*>(xp), rsc, M, K, RT, *na);
  else
    hipLaunchKernelGGL(pack_x_kernel<false>, dim3(16 * RT), dim3(kSplitThreads), 0, st, x,
                       reinterpret_cast<uint2*>(xp), rsc, M, K, RT, NormArgs{});
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  auto kern = dgemm_kernel<RT, kDgT, kDgW, dg_depth(RT)>;
  constexpr size_t lds = static_cast<size_t>(dg_depth(RT)) * RT * 4 * kWave * 16 +
                        static_cast<size_t>(kDgCols) * (kDgScaleGroups + 1) * sizeof(float);
  static std::atomic<uint64_t> done{0};
  if (lds > 64 * 1024) {
    e = ensure_dynamic_lds(reinterpret_cast<const void*>(kern), lds, done);
    if (e != hipSuccess) return e;
  }
  const int cols = epi.mode == kEpiSwiglu ? (N / 2 + kDgCols / 2 - 1) / (kDgCols / 2)
                                          : (N + kDgCols - 1) / kDgCols;
  float* out = p.splits > 1 ? part : y;
  hipLaunchKernelGGL(kern, dim3(cols, p.splits), dim3(kDgW * kWave), lds, st, xp, rsc, w, s,
                     out, M, N, K, gs, p.groups_per_split, epi, pk);
  e = hipGetLastError();
  if (e != hipSuccess || p.splits == 1) return e;
  const size_t count = static_cast<size_t>(M) * (epi.mode == kEpiSwiglu ? N / 2 : N);
  const int grid = static_cast<int>(std::min<size_t>((count + kThreads - 1) / kThreads, 4096));
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(grid), dim3(kThreads), 0, st, part, y, M, N,
                     p.splits, epi);
  return hipGetLastError();
}

template <int RT, int T, int W>
hipError_t launch_tile(const float* x, const int8_t* w, const float* s, float* y, void* ws, int M,
                       int N, int K, int gs, const Plan& p, hipStream_t st,
                       const NormArgs* na, int pk) {
  unsigned* tickets = static_cast<unsigned*>(ws);
  char* base = static_cast<char*>(ws) + kTicketBytes;
  u32x4* xp = reinterpret_cast<u32x4*>(base);
  base += align256(static_cast<size_t>(K / BK) * RT * 4 * kWave * sizeof(u32x4));
  float* rsc = reinterpret_cast<float*>(base);
  base += align256(static_cast<size_t>(16 * RT) * sizeof(float));
  float* part = reinterpret_cast<float*>(base);
  if (na)
    hipLaunchKernelGGL(pack_x_kernel<true>, dim3(16 * RT), dim3(kSplitThreads), 0, st, x,
                       reinterpret_cast<uint2*>(xp), rsc, M, K, RT, *na);
  else
    hipLaunchKernelGGL(pack_x_kernel<false>, dim3(16 * RT), dim3(kSplitThreads), 0, st, x,
                       reinterpret_cast<uint2*>(xp), rsc, M, K, RT, NormArgs{});
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const dim3 grid((N + 16 * T - 1) / (16 * T), p.splits);
  hipLaunchKernelGGL((tile_kernel<RT, T, W>), grid, dim3(W * kWave), 0, st, xp, rsc, w, s,
                     y, part, tickets, M, N, K, gs, p.groups_per_split, p.splits, pk);
  return hipGetLastError();
}

// ---------------------------------------------------------------- packed GEMV (1-2 rows)
// Weights in the packed layout (lane_wbase). Workgroups are resident for the whole call: each
// stages x (MT rows of K floats) in LDS once, then its waves walk units in grid stride, with
// no further barrier. A unit is one 16-row tile and a contiguous slice of KS groups (a KS KiB
// run of the packed weights); a wave issues U KiB of it per step before using any (latency is
// hidden by residency, as in the row-major GEMV), and the row's scales of 4 groups arrive as
// one float4. Per group a lane holds 16 weights of row lane % 16 at k = 64 g + 16 (lane / 16)
// and multiplies them with the matching 16 activations (float4 LDS reads shared by the 16 lanes
// of a quarter). The four quarters' sums are added with two lane swaps. With S > 1 slices per
// tile, each unit stores its 16 x MT sums as a partial and takes a ticket; the last unit of the
// tile sums the S partials in slice order and resets the ticket.

template <int MT, int U>
__global__ __launch_bounds__(kPgWaves * kWave) void pgemv_kernel(
    const float* __restrict__ x, const int8_t* w, const float* __restrict__ s,
    float* __restrict__ y, float* __restrict__ part, unsigned* __restrict__ tickets, int M, int N,
    int K, int ks, int S) {
  static_assert(U % 4 == 0, "scales are read as whole float4s");
  extern __shared__ __attribute__((aligned(16))) float4 xs[];  // [MT][K / 4]
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lcol = lane & 15, q = lane >> 4;
  const int G = K / BK;
  const int K4 = K / 4;
  for (int c = tid; c < MT * K4; c += kPgWaves * kWave)
    xs[c] = *reinterpret_cast<const float4*>(x + ix::pg_xsrc(c, K4, M, K));
  __syncthreads();

  const int ntiles = (N + 15) / 16;
  const int units = ntiles * S;
  for (int u = blockIdx.x * kPgWaves + wave; u < units; u += gridDim.x * kPgWaves) {
    const int tile = u / S, sl = u - tile * S;
    const int g0 = sl * ks, gn = min(ks, G - g0);
    const int8_t* wb = w + ix::pg_wbase(tile, K, g0, lane);
    const float* sr = s + ix::pg_srow(tile, lcol, N, G, g0);
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.f;
    for (int i0 = 0; i0 < gn; i0 += U) {
      u32x4 wq[U];
      float sc[U];
#pragma unroll
      for (int v = 0; v < U; ++v)
        wq[v] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(wb + static_cast<size_t>(ix::pg_wslot(i0, v, gn)) * 1024));
#pragma unroll
      for (int v = 0; v < U; v += 4) {
        // gn % 4 == 0 (K % 256 == 0, ks % 4 == 0): slots past gn get scale 0 below.
        const float4 f = *reinterpret_cast<const float4*>(sr + ix::pg_sslot(i0, v, gn));
        sc[v] = f.x;
        sc[v + 1] = f.y;
        sc[v + 2] = f.z;
        sc[v + 3] = f.w;
      }
#pragma unroll
      for (int v = 0; v < U; ++v) {
        __builtin_amdgcn_sched_barrier(0);  // one group's LDS reads at a time
        const i32x4 wv = __builtin_bit_cast(i32x4, wq[v]);
        const int k4 = (g0 + ix::pg_wslot(i0, v, gn)) * 16 + q * 4;
        const float scv = i0 + v < gn ? sc[v] : 0.f;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          const float4* xp = &xs[m * K4 + k4];
          acc[m] = fmaf(scv, dot16(wv, xp[0], xp[1], xp[2], xp[3]), acc[m]);
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      acc[m] += __shfl_xor(acc[m], 16, kWave);
      acc[m] += __shfl_xor(acc[m], 32, kWave);
    }
    const int n = tile * 16 + lcol;
    if (S == 1) {
#pragma unroll
      for (int m = 0; m < MT; ++m)
        if (lane < 16 && m < M && n < N) y[static_cast<size_t>(m) * N + n] = acc[m];
      continue;
    }
#pragma unroll
    for (int m = 0; m < MT; ++m)
      if (lane < 16 && m < M && n < N)
        __hip_atomic_store(part + ix::pg_part(sl, M, m, N, n), acc[m],
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // The last unit of the tile sums the slices in order.
    publish_partials();
    unsigned t = 0;
    if (lane == 0)
      t = __hip_atomic_fetch_add(&tickets[tile], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    t = __shfl(t, 0, kWave);
    if (t != static_cast<unsigned>(S - 1)) continue;
    acquire_partials();
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (lane < 16 && m < M && n < N) {
        float v = 0.f;
        for (int z = 0; z < S; ++z)
          v += __hip_atomic_load(part + ix::pg_part(z, M, m, N, n),
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        y[static_cast<size_t>(m) * N + n] = v;
      }
    }
    if (lane == 0)
      __hip_atomic_store(&tickets[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

PgPlan pgemv_plan(int M, int N, int K) {
  return pgemv_plan_for(M, N, K, cu_count(), SQ8_PGEMV_WPC);
}

template <int MT>
hipError_t launch_pgemv_mt(const float* x, const int8_t* w, const float* s, float* y, void* ws,
                           int M, int N, int K, hipStream_t st) {
  const PgPlan p = pgemv_plan(MT, N, K);
  auto kern = pgemv_kernel<MT, SQ8_PGEMV_U>;
  static std::atomic<uint64_t> done{0};
  if (p.lds > 64 * 1024) {
    if (p.lds > 144 * 1024) return hipErrorInvalidValue;
    const hipError_t e = ensure_dynamic_lds(reinterpret_cast<const void*>(kern), 144 * 1024, done);
    if (e != hipSuccess) return e;
  }
  unsigned* tickets = static_cast<unsigned*>(ws);
  float* part = reinterpret_cast<float*>(static_cast<char*>(ws) + kTicketBytes);
  hipLaunchKernelGGL(kern, dim3(p.grid), dim3(kPgWaves * kWave), p.lds, st, x, w, s, y, part,
                     tickets, M, N, K, p.ks, p.S);
  return hipGetLastError();
}

bool pgemv_ok(int M, int K, int gs, const float* s) {
  return pgemv_ok_for(M, K, gs, (reinterpret_cast<uintptr_t>(s) & 15) == 0);
}

hipError_t launch_pgemv(const float* x, const int8_t* w, const float* s, float* y, void* ws,
                        int M, int N, int K, hipStream_t st) {
  switch (M) {
    case 1: return launch_pgemv_mt<1>(x, w, s, y, ws, M, N, K, st);
    default: return launch_pgemv_mt<2>(x, w, s, y, ws, M, N, K, st);
  }
}

}  // namespace

// Workspace layout: [ticket array, kTicketBytes][path buffers]. The ticket array must be zero
// before the first call; every call leaves it zero.
size_t mfma_workspace_bytes(int M, int N, int K) {
  const Plan p = make_plan(M, N, K);
  size_t b = kTicketBytes;
  if (p.tile || p.dgemm) {
    b += align256(static_cast<size_t>(K / BK) * p.rt * 4 * kWave * sizeof(u32x4));
    b += align256(static_cast<size_t>(16 * p.rt) * sizeof(float));
  } else if (!p.skinny) {
    b += 2 * align256(static_cast<size_t>(M) * K * sizeof(_Float16));
    b += align256(static_cast<size_t>(M) * sizeof(float));
  }
  if (p.splits > 1) b += align256(static_cast<size_t>(p.splits) * M * N * sizeof(float));
  return b;
}

// Requires: K % 64 == 0, group_size % 64 == 0, K % group_size == 0, 16-byte aligned x and w,
// workspace of mfma_workspace_bytes(M, N, K).
bool mfma_fuses_epilogue(int M, int N, int K) {
  const Plan p = make_plan(M, N, K);
  return !p.tile && !p.skinny;  // the GEMM and the decode GEMM
}

hipError_t launch_epilogue(const float* t, float* y, int M, int N, Epi epi, hipStream_t st) {
  const size_t count = static_cast<size_t>(M) * (epi.mode == kEpiSwiglu ? N / 2 : N);
  const int grid = static_cast<int>(std::min<size_t>((count + kThreads - 1) / kThreads, 4096));
  hipLaunchKernelGGL(epilogue_kernel, dim3(grid), dim3(kThreads), 0, st, t, y, M, N, epi);
  return hipGetLastError();
}

bool mfma_norm_fused(int M, int N, int K) {
  const Plan p = make_plan(M, N, K);
  return (p.tile || p.dgemm) && K % 4 == 0 && K <= kSplitThreads * 4 * kSplitV;
}

// Packed weight layout (lane_wbase): 16-byte unit d of the packed buffer is lane L = d % 64 of
// group g = (d / 64) % G of tile t = d / (64 G): row 16 t + L % 16, bytes 64 g + 16 (L / 16) ..
// +15 of that row, zero for the padding rows past N. Reads are 64-byte runs of 16 rows, writes
// are contiguous.
__global__ __launch_bounds__(kThreads) void pack_weights_kernel(const int8_t* __restrict__ w,
                                                                int N, int K,
                                                                u32x4* __restrict__ wp,
                                                                size_t units) {
  const int G = K / BK;
  for (size_t d = blockIdx.x * static_cast<size_t>(kThreads) + threadIdx.x; d < units;
       d += static_cast<size_t>(gridDim.x) * kThreads) {
    const int L = static_cast<int>(d & 63);
    const size_t tg = d >> 6;
    const int g = static_cast<int>(tg % G);
    const size_t row = (tg / G) * 16 + (L & 15);
    u32x4 v = {0u, 0u, 0u, 0u};
    if (row < static_cast<size_t>(N))
      v = *reinterpret_cast<const u32x4*>(w + row * K + g * BK + (L >> 4) * 16);
    wp[d] = v;
  }
}

hipError_t launch_pack_weights(const int8_t* w, int N, int K, int8_t* wp, hipStream_t st) {
  const size_t units = static_cast<size_t>((N + 15) / 16) * 16 * K / 16;
  const int grid = static_cast<int>(std::min<size_t>((units + kThreads - 1) / kThreads, 8192));
  hipLaunchKernelGGL(pack_weights_kernel, dim3(grid), dim3(kThreads), 0, st, w, N, K,
                     reinterpret_cast<u32x4*>(wp), units);
  return hipGetLastError();
}

bool mfma_packed_ok(int M, int N, int K) { return M > 0 && N > 0 && K > 0; }

// Either path's need: whether the GEMV serves a call also depends on the scales' alignment.
size_t packed_workspace_bytes(int M, int N, int K, int gs) {
  const size_t b = mfma_workspace_bytes(M, N, K);
  if (!pgemv_ok(M, K, gs, nullptr)) return b;
  const PgPlan p = pgemv_plan(M, N, K);
  size_t g = kTicketBytes;
  if (p.S > 1) g += align256(static_cast<size_t>(p.S) * M * N * sizeof(float));
  return std::max(b, g);
}

hipError_t launch_mfma(const float* x, const int8_t* w, const float* s, float* y, int M, int N,
                       int K, int gs, void* ws, hipStream_t st, Epi epi, const NormArgs* na,
                       int pk) {
  if (pk && pgemv_ok(M, K, gs, s)) {
    if (epi.mode != kEpiNone || na) return hipErrorInvalidValue;
    return launch_pgemv(x, w, s, y, ws, M, N, K, st);
  }
  const Plan p = make_plan(M, N, K);
  if (epi.mode != kEpiNone && (p.tile || p.skinny)) return hipErrorInvalidValue;
  if (na && !mfma_norm_fused(M, N, K)) return hipErrorInvalidValue;
  if (p.dgemm) {
    switch (p.rt) {
      case 1: return launch_dgemm<1>(x, w, s, y, ws, M, N, K, gs, p, st, epi, na, pk);
      case 2: return launch_dgemm<2>(x, w, s, y, ws, M, N, K, gs, p, st, epi, na, pk);
      case 3: return launch_dgemm<3>(x, w, s, y, ws, M, N, K, gs, p, st, epi, na, pk);
      default: return launch_dgemm<4>(x, w, s, y, ws, M, N, K, gs, p, st, epi, na, pk);
    }
  }
  unsigned* tickets = static_cast<unsigned*>(ws);
  char* base = static_cast<char*>(ws) + kTicketBytes;
  if (p.tile) {
    const int key = p.rt * 100 + p.tn * 10 + (p.tw >= 8 ? 8 : p.tw);
    switch (key) {
      case 128: return launch_tile<1, 2, 8>(x, w, s, y, ws, M, N, K, gs, p, st, na, pk);
      case 144: return launch_tile<1, 4, 4>(x, w, s, y, ws, M, N, K, gs, p, st, na, pk);
      case 228: return launch_tile<2, 2, 8>(x, w, s, y, ws, M, N, K, gs, p, st, na, pk);
      case 244: return launch_tile<2, 4, 4>(x, w, s, y, ws, M, N, K, gs, p, st, na, pk);
      case 328: return launch_tile<3, 2, 8>(x, w, s, y, ws, M, N, K, gs, p, st, na, pk);
      case 342: return launch_tile<3, 4, 2>(x, w, s, y, ws, M, N, K, gs, p, st, na, pk);
      case 428: return launch_tile<4, 2, 8>(x, w, s, y, ws, M, N, K, gs, p, st, na, pk);
      case 442: return launch_tile<4, 4, 2>(x, w, s, y, ws, M, N, K, gs, p, st, na, pk);
      default: return hipErrorInvalidValue;
    }
  }
  if (p.skinny) {
    float* part = reinterpret_cast<float*>(base);
#define SQ8_SKINNY(MR, MT16)                                                               \
  switch (p.kw) {                                                                          \
    case 4: return launch_skinny16<MR, 4, 1, MT16>(x, w, s, y, part, tickets, M, N, K, gs, p, st, pk); \
    case 2: return launch_skinny16<MR, 2, 1, MT16>(x, w, s, y, part, tickets, M, N, K, gs, p, st, pk); \
    default: return launch_skinny16<MR, 1, 1, MT16>(x, w, s, y, part, tickets, M, N, K, gs, p, st, pk); \
  }
    if (M <= 4) {  // int8-limb MFMA kernel: one MFMA covers 4 tokens
      if (p.kw == 4) return launch_skinny_i8<1, 4, 1>(x, w, s, y, part, tickets, M, N, K, gs, p, st, pk);
      if (p.kw == 2) return launch_skinny_i8<1, 2, 1>(x, w, s, y, part, tickets, M, N, K, gs, p, st, pk);
      return launch_skinny_i8<1, 1, 1>(x, w, s, y, part, tickets, M, N, K, gs, p, st, pk);
    }
    if (M <= 8 && p.kw == 4)
      return launch_skinny16<8, 4, 1, 1>(x, w, s, y, part, tickets, M, N, K, gs, p, st, pk);
    if (M <= 8 && p.kw == 2)
      return launch_skinny16<8, 2, 1, 1>(x, w, s, y, part, tickets, M, N, K, gs, p, st, pk);
    if (M <= 16) SQ8_SKINNY(16, 1);
    if (M <= 32) SQ8_SKINNY(32, 2);
    if (M <= 48) SQ8_SKINNY(48, 3);
    SQ8_SKINNY(64, 4);
#undef SQ8_SKINNY
  }
  _Float16* xh = reinterpret_cast<_Float16*>(base);
  base += align256(static_cast<size_t>(M) * K * sizeof(_Float16));
  _Float16* xl = reinterpret_cast<_Float16*>(base);
  base += align256(static_cast<size_t>(M) * K * sizeof(_Float16));
  float* rsc = reinterpret_cast<float*>(base);
  base += align256(static_cast<size_t>(M) * sizeof(float));
  float* part = p.splits > 1 ? reinterpret_cast<float*>(base) : y;

  hipLaunchKernelGGL(split_x_kernel, dim3(M), dim3(kSplitThreads), 0, st, x, xh, xl, rsc, K);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (p.cfg == 1)
    e = p.gps == 1
            ? launch_gemm<1, 4, 2, 2, 3>(xh, xl, rsc, w, s, part, M, N, K, gs, p, st, epi, pk)
            : launch_gemm<2, 4, 1, 2, 2, 2>(xh, xl, rsc, w, s, part, M, N, K, gs, p, st, epi, pk);
  else
    e = launch_gemm<2, 4, 2, 2, 3>(xh, xl, rsc, w, s, part, M, N, K, gs, p, st, epi, pk);
  if (e != hipSuccess || p.splits == 1) return e;
  const size_t count = static_cast<size_t>(M) * (epi.mode == kEpiSwiglu ? N / 2 : N);
  const int grid = static_cast<int>(std::min<size_t>((count + kThreads - 1) / kThreads, 4096));
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(grid), dim3(kThreads), 0, st, part, y, M, N,
                     p.splits, epi);
  return hipGetLastError();
}

}  // namespace sq8
