// Bandwidth-bound decode kernels (few token rows) for gfx950.
//
// Reference behaviour replaced: matmul_kernel_cu_fp32int8<128> (matmul_kernel.cu:65-99), one
// 128-thread block per output row with 1-byte scalar weight loads, a per-element scale gather and
// a cub block reduction per (row, token).
//
// Two kernels:
//  - sweep_kernel (M <= 4, the decode GEMV): the token rows are staged once per workgroup in
//    LDS; each wave takes row blocks of R rows in grid stride and walks K in steps of U KiB per
//    row. Latency is hidden by residency (up to 16 waves per CU) and by the compiler's
//    interleaving of a step's loads with its dot products; only the group scales are fetched a
//    step ahead. Each lane converts its 16 int8 per row with SDWA byte-select conversions and
//    applies the group scale once per 16-element chunk.
//  - gemv_rows_kernel (fallback for larger M or K beyond the LDS budget):
// a 256-thread workgroup (4 wave64s) owns R consecutive output rows and the whole K
// extent. Every lane streams 16 int8 weights per row per step with one dwordx4 load; the 256 lanes
// of a workgroup cover 4 KiB of each row per step, fully coalesced. A 16-byte chunk never straddles
// a K-group (group_size % 16 == 0), so the lane applies its group scale once per chunk after a
// 16-term fp32 dot product. The R x MT partial sums of a lane are reduced across the wave with a
// reduce-scatter butterfly (R*MT values in log2(R*MT) exchange rounds instead of 6 rounds each),
// then across the 4 waves through LDS in a fixed order, so results are deterministic.
#include <cmath>

#include "sq8_common.h"

namespace sq8 {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

// Reduce NV per-lane values over the 64 lanes of a wave. On return v[0] of lane l holds the
// wave-wide sum of value index (l >> (6 - log2 NV)). Every value is summed in the same pairing
// order (xor 32, 16, 8, 4, 2, 1) whatever NV is, so the result of a (row, token) pair does not
// depend on how many tokens share the launch.
template <int NV>
__device__ __forceinline__ void wave_reduce_scatter(float (&v)[NV], int lane) {
  static_assert((NV & (NV - 1)) == 0 && NV <= 64, "NV must be a power of two <= 64");
  int off = 32;
#pragma unroll
  for (int half = NV / 2; half >= 1; half /= 2, off /= 2) {
    const bool upper = (lane & off) != 0;
#pragma unroll
    for (int i = 0; i < half; ++i) {
      const float send = upper ? v[i] : v[i + half];
      const float keep = upper ? v[i + half] : v[i];
      v[i] = keep + __shfl_xor(send, off, kWave);
    }
  }
#pragma unroll
  for (; off >= 1; off /= 2) v[0] += __shfl_xor(v[0], off, kWave);
}

// R rows per workgroup, MT token rows per pass, GS = group size (0: runtime value, multiple of 16).
template <int R, int MT, int GS>
__global__ __launch_bounds__(kThreads) void gemv_rows_kernel(const float* __restrict__ x,
                                                             const int8_t* __restrict__ w,
                                                             const float* __restrict__ s,
                                                             float* __restrict__ y, int M, int N,
                                                             int K, int gs_rt) {
  constexpr int NV = R * MT;
  __shared__ float red[kWaves][NV];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar address math
  const int n0 = blockIdx.x * R;
  const int gs = GS ? GS : gs_rt;
  const int chunks_per_group = gs >> 4;
  const int nchunk = K >> 4;
  const int groups_per_row = K / gs;

  // Rows past N are clamped to the last row (loads stay in bounds); their sums are not stored.
  const i32x4* wrow[R];
  const float* srow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int n = min(n0 + r, N - 1);
    wrow[r] = reinterpret_cast<const i32x4*>(w + static_cast<size_t>(n) * K);
    srow[r] = s + static_cast<size_t>(n) * groups_per_row;
  }

  for (int m0 = 0; m0 < M; m0 += MT) {
    const float4* xrow[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = min(m0 + t, M - 1);
      xrow[t] = reinterpret_cast<const float4*>(x + static_cast<size_t>(m) * K);
    }
    float acc[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) acc[i] = 0.f;

#pragma unroll 2
    for (int c = tid; c < nchunk; c += kThreads) {
      const int g = GS ? (c / ((GS > 0 ? GS : 16) / 16)) : (c / chunks_per_group);
      i32x4 q[R];
      float sc[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        q[r] = __builtin_nontemporal_load(wrow[r] + c);
        sc[r] = srow[r][g];
      }
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const float4 x0 = xrow[t][4 * c + 0];
        const float4 x1 = xrow[t][4 * c + 1];
        const float4 x2 = xrow[t][4 * c + 2];
        const float4 x3 = xrow[t][4 * c + 3];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          acc[r * MT + t] = fmaf(sc[r], dot16(q[r], x0, x1, x2, x3), acc[r * MT + t]);
        }
      }
    }

    wave_reduce_scatter<NV>(acc, lane);
    constexpr int kSpan = kWave / NV;  // lanes that end up holding the same value index
    if ((lane & (kSpan - 1)) == 0) red[wave][lane / kSpan] = acc[0];
    __syncthreads();
    if (tid < NV) {
      const int r = tid / MT, t = tid % MT;
      float v = red[0][tid];
#pragma unroll
      for (int wv = 1; wv < kWaves; ++wv) v += red[wv][tid];
      const int n = n0 + r, m = m0 + t;
      if (n < N && m < M) y[static_cast<size_t>(m) * N + n] = v;
    }
    __syncthreads();
  }
}

// Decode GEMV. M <= MT token rows (padded with zero rows to MT) are staged in LDS once per
// workgroup; wave w of the grid takes row blocks w, w + GW, ... of R rows and walks K in steps of
// U KiB per row, issuing all R x U dwordx4 loads of a step before using any of them. Latency is
// hidden by residency (four 4-wave workgroups per CU) rather than by a second register set, which
// keeps the register count low enough for that residency. TAIL: K is not a multiple of U KiB.
// Optional work done while staging a single token row (M = 1), fusing the decode step's
// elementwise layers into the projection that consumes them:
//   kProNorm:   x' = x + res (res may be null), staged value rmsnorm(x') * nw; workgroup 0 also
//               writes x' to x_out (may be null) as the new residual stream;
//   kProSwiGLU: x holds [a | b] (2K values); staged value silu(a) * b.
enum Prologue { kProNone = 0, kProNorm = 1, kProSwiGLU = 2 };
// silu(a) * b as the reference's SwiGLU computes it (swiglu_kernel.cu:12-19).
__device__ __forceinline__ float silu_mul(float a, float b) {
  const float sig = 1.0f / (1.0f + expf(-a));
  return (a * sig) * b;
}
struct ProArgs {
  const float* res;
  float* x_out;
  const float* nw;
  float eps;
};

// Stage the token rows (or the fused prologue's result) in LDS for a workgroup of WV waves.
// Token rows M .. MT-1 are staged as zeros. float4 number i is stored at i ^ ((i >> 4) & 3): a
// lane reads the 4 float4 of its 16-element chunk, and without the swizzle lanes l and l+4 would
// hit the same LDS banks in every ds_read_b128 (4-way conflicts). The caller's barrier publishes
// the stage.
// kProNorm stages r * nw (r = x + res) in the same single pass that sums r^2: the RMSNorm scale
// rsqrt(mean(r^2) + eps) is a scalar of the row, so it multiplies the finished dot products
// instead of every staged value, and the stage needs no reduction barrier of its own. The
// per-wave sums of squares are left in the returned LDS array for norm_scale() after the barrier.
template <int MT, int WV, int PRO>
__device__ __forceinline__ const float* stage_x(const float* __restrict__ x, int M, int K,
                                                const ProArgs& pro, float* xs) {
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const float4* x4 = reinterpret_cast<const float4*>(x);
  float4* xs4 = reinterpret_cast<float4*>(xs);
  if (PRO == kProNone) {
    for (int i = tid; i < MT * K / 4; i += WV * kWave) {
      const float4 v = i < M * K / 4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
      xs4[i ^ ((i >> 4) & 3)] = v;
    }
    return nullptr;
  } else if (PRO == kProNorm) {
    __shared__ float red[WV];
    const float4* r4 = reinterpret_cast<const float4*>(pro.res);
    const float4* n4 = reinterpret_cast<const float4*>(pro.nw);
    float4* o4 = reinterpret_cast<float4*>(pro.x_out);
    float ss = 0.f;
    for (int i = tid; i < K / 4; i += WV * kWave) {
      float4 v = x4[i];
      if (r4) {
        const float4 r = r4[i];
        v = make_float4(v.x + r.x, v.y + r.y, v.z + r.z, v.w + r.w);
      }
      if (o4 && blockIdx.x == 0) o4[i] = v;
      ss = fmaf(v.x, v.x, ss);
      ss = fmaf(v.y, v.y, ss);
      ss = fmaf(v.z, v.z, ss);
      ss = fmaf(v.w, v.w, ss);
      const float4 g = n4[i];
      xs4[i ^ ((i >> 4) & 3)] = make_float4(v.x * g.x, v.y * g.y, v.z * g.z, v.w * g.w);
    }
#pragma unroll
    for (int off = 32; off >= 1; off /= 2) ss += __shfl_xor(ss, off, kWave);
    if (lane == 0) red[wave] = ss;
    return red;
  } else {
    for (int i = tid; i < K / 4; i += WV * kWave) {
      const float4 a = x4[i], g = x4[K / 4 + i];
      xs4[i ^ ((i >> 4) & 3)] = make_float4(silu_mul(a.x, g.x), silu_mul(a.y, g.y),
                                            silu_mul(a.z, g.z), silu_mul(a.w, g.w));
    }
    return nullptr;
  }
}

// The RMSNorm scale of the staged row (after the barrier that published stage_x's sums): the
// waves' sums of squares are added in wave order, so every workgroup gets the same value.
template <int WV>
__device__ __forceinline__ float norm_scale(const float* red, int K, float eps) {
  float total = red[0];
#pragma unroll
  for (int v = 1; v < WV; ++v) total += red[v];
  return rsqrtf(total / static_cast<float>(K) + eps);
}

// Rows of block b: R consecutive rows, or with PAIR (R = 2, a fused [gate; up] weight of N = 2F
// rows) the gate row b and its up row b + F, so that one wave holds both dot products of a
// SwiGLU output. Blocks past the last read row N - 1 (their results are dropped).
template <int R, bool PAIR>
__device__ __forceinline__ int block_row(int b, int r, int N) {
  return PAIR ? min(b + r * (N / 2), N - 1) : min(b * R + r, N - 1);
}

// With PAIR (M = 1, R = 2) the kernel writes y[b] = silu(g) * u for the row pair of block b
// (the SwiGLU of a fused [gate; up] projection, N/2 outputs) instead of the two rows.
template <int R, int U, int MT, int GS, bool TAIL, int WV = kWaves, int PRO = kProNone,
          bool PAIR = false>
__global__ __launch_bounds__(WV * kWave) void sweep_kernel(const float* __restrict__ x,
                                                         const int8_t* __restrict__ w,
                                                         const float* __restrict__ s,
                                                         float* __restrict__ y, int M, int N,
                                                         int K, int gs_rt, ProArgs pro = {}) {
  extern __shared__ float xs[];
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar address math
  static_assert(!PAIR || (R == 2 && MT == 1), "row pairs: two rows, one token");
  const int nblk = PAIR ? N / 2 : (N + R - 1) / R;
  const int GW = gridDim.x * WV;
  const int gs = GS ? GS : gs_rt;
  const int gpr = K / gs;
  const int nsteps = (K + 1024 * U - 1) / (1024 * U);
  // The scales of a step are loaded one step ahead. Needed only after the dot products, they would
  // otherwise be scheduled after them and add a second memory round trip to every step. Rows
  // past N (including those of a block past the last) are clamped to row N - 1.
  auto load_scales = [&](int b, int st, float (&sc)[U][R]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = (st * U + u) * 1024 + lane * 16;
      const int kc = !TAIL || k < K ? k : 0;
#pragma unroll
      for (int r = 0; r < R; ++r)
        sc[u][r] = s[static_cast<size_t>(block_row<R, PAIR>(b, r, N)) * gpr + kc / gs];
    }
  };
  auto load_w = [&](int b, int st, i32x4 (&q)[U][R]) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = (st * U + u) * 1024 + lane * 16;
      const bool ok = !TAIL || k < K;
      const int kc = ok ? k : 0;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int n = block_row<R, PAIR>(b, r, N);
        const i32x4 v = __builtin_nontemporal_load(
            reinterpret_cast<const i32x4*>(w + static_cast<size_t>(n) * K + kc));
        q[u][r] = ok ? v : i32x4{0, 0, 0, 0};
      }
    }
  };
  // With a fused prologue (RMSNorm, SwiGLU) the first step's weights and scales are requested
  // before the activations are staged, so their memory latency overlaps the two-pass staging
  // and its barriers instead of following them (+2.6 % decode tokens/s on MI355X). For a plain
  // copy of x the staging is short and the early requests measured slower on the decode step,
  // so there the weights are requested after it. Waves without a block (the tail of the last
  // workgroup) read row N - 1 and discard it.
  constexpr bool kEarly = PRO != kProNone;
  int b = blockIdx.x * WV + wave, st = 0;
  i32x4 q[U][R];
  float scn[U][R];
  if constexpr (kEarly) {
    load_w(b, 0, q);
    load_scales(b, 0, scn);
  }

  const float* red = stage_x<MT, WV, PRO>(x, M, K, pro, xs);
  __syncthreads();
  if constexpr (!kEarly) load_scales(b, 0, scn);
  const float rs = PRO == kProNorm ? norm_scale<WV>(red, K, pro.eps) : 1.f;

  float acc[R * MT];
#pragma unroll
  for (int i = 0; i < R * MT; ++i) acc[i] = 0.f;
  auto step = [&]() __attribute__((always_inline)) {
    float sc[U][R];
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int r = 0; r < R; ++r) sc[u][r] = scn[u][r];
    int b1 = b, st1 = st + 1;
    if (st1 == nsteps) { st1 = 0; b1 += GW; }
    load_scales(b1, st1, scn);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = (st * U + u) * 1024 + lane * 16;
      const int kc = !TAIL || k < K ? k : 0;
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        const int i0 = (t * K + kc) / 4;
        const float4* xp = reinterpret_cast<const float4*>(xs) + i0;
        const int sw = (i0 >> 4) & 3;
        const float4 x0 = xp[0 ^ sw], x1 = xp[1 ^ sw], x2 = xp[2 ^ sw], x3 = xp[3 ^ sw];
#pragma unroll
        for (int r = 0; r < R; ++r)
          acc[r * MT + t] = fmaf(sc[u][r], dot16(q[u][r], x0, x1, x2, x3), acc[r * MT + t]);
      }
    }
    if (st == nsteps - 1) {
      wave_reduce_scatter<R * MT>(acc, lane);
      constexpr int kSpan = kWave / (R * MT);
      if constexpr (PAIR) {
        const float u = __shfl(acc[0], kSpan, kWave);  // the up row's sum (value index 1)
        if (lane == 0 && b < nblk) y[b] = silu_mul(acc[0] * rs, u * rs);
      } else if ((lane & (kSpan - 1)) == 0) {
        const int idx = lane / kSpan, r = idx / MT, t = idx % MT;
        const int n = b * R + r;
        if (n < N && t < M) y[static_cast<size_t>(t) * N + n] = PRO == kProNorm ? acc[0] * rs
                                                                               : acc[0];
      }
#pragma unroll
      for (int i = 0; i < R * MT; ++i) acc[i] = 0.f;
    }
    b = b1;
    st = st1;
  };
  if constexpr (kEarly) {
    if (b < nblk) step();  // first step: weights already requested
  }
  while (b < nblk) {
    load_w(b, st, q);
    step();
  }
}

// Single-token GEMV for few, long rows (N small, K >= 8 KiB): a workgroup of WV waves owns
// WV/KS rows and the KS waves of a row split its 1 KiB chunks (wave part p takes chunks p, p + KS,
// ..., so neighbouring waves read neighbouring pieces of the row). A wave requests all of its U
// chunks (and their scales) at once, then the row's KS partial sums are added in LDS in part
// order. With one row per wave, such a shape leaves most of the chip idle and every wave walks
// its row in several dependent round trips.
template <int U, int KS, int WV, int GS, bool TAIL, int PRO>
__global__ __launch_bounds__(WV * kWave) void splitrow_kernel(const float* __restrict__ x,
                                                            const int8_t* __restrict__ w,
                                                            const float* __restrict__ s,
                                                            float* __restrict__ y, int N, int K,
                                                            int gs_rt, ProArgs pro) {
  static_assert(WV % KS == 0, "whole rows per workgroup");
  constexpr int RW = WV / KS;
  extern __shared__ float xs[];
  __shared__ float part[WV];
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rw = wave / KS, p = wave % KS;
  const int nr = min(blockIdx.x * RW + rw, N - 1);
  const int gs = GS ? GS : gs_rt;
  const int8_t* wrow = w + static_cast<size_t>(nr) * K;
  const float* srow = s + static_cast<size_t>(nr) * (K / gs);
  i32x4 q[U];
  float sc[U];
  // Chunks past the row end (TAIL) read the row's first chunk and are dropped at use.
  auto issue = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = (p + KS * u) * 1024 + lane * 16;
      const int kc = !TAIL || k < K ? k : 0;
      q[u] = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(wrow + kc));
      sc[u] = srow[kc / gs];
    }
  };
  // Behind a fused prologue the weights are requested first (their latency overlaps the
  // staging); with a plain copy of x they follow it, as in sweep_kernel.
  constexpr bool kEarly = PRO != kProNone;
  if constexpr (kEarly) issue();
  const float* red = stage_x<1, WV, PRO>(x, 1, K, pro, xs);
  __syncthreads();
  if constexpr (!kEarly) issue();
  const float rs = PRO == kProNorm ? norm_scale<WV>(red, K, pro.eps) : 1.f;
  float acc = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int k = (p + KS * u) * 1024 + lane * 16;
    const bool ok = !TAIL || k < K;
    const int i0 = (ok ? k : 0) / 4;
    const float4* xp = reinterpret_cast<const float4*>(xs) + i0;
    const int sw = (i0 >> 4) & 3;
    const float4 x0 = xp[0 ^ sw], x1 = xp[1 ^ sw], x2 = xp[2 ^ sw], x3 = xp[3 ^ sw];
    const float d = dot16(q[u], x0, x1, x2, x3);
    acc = fmaf(ok ? sc[u] : 0.f, d, acc);
  }
#pragma unroll
  for (int off = 32; off >= 1; off /= 2) acc += __shfl_xor(acc, off, kWave);
  if (lane == 0) part[wave] = acc;
  __syncthreads();
  if (tid < RW) {
    float v = part[tid * KS];
#pragma unroll
    for (int i = 1; i < KS; ++i) v += part[tid * KS + i];
    const int n = blockIdx.x * RW + tid;
    if (n < N) y[n] = PRO == kProNorm ? v * rs : v;
  }
}

// Exact restatement of the reference indexing for any group size and any K % 4 == 0, used when
// the fast path's alignment or group-size assumptions do not hold: scale of (n, k) is
// scales[(n*K)/gs + k/gs] (matmul_kernel.cu:77,86). One workgroup per (row, token).
__global__ __launch_bounds__(kThreads) void generic_kernel(const float* __restrict__ x,
                                                          const int8_t* __restrict__ w,
                                                          const float* __restrict__ s,
                                                          float* __restrict__ y, int M, int N,
                                                          int K, int gs) {
  __shared__ float red[kWaves];
  const int n = blockIdx.x;
  const int m = blockIdx.y;
  const int tid = threadIdx.x;
  const int8_t* wr = w + static_cast<size_t>(n) * K;
  const float* sr = s + (static_cast<int64_t>(n) * K) / gs;
  const float* xr = x + static_cast<size_t>(m) * K;
  float acc = 0.f;
  for (int k = tid; k < K; k += kThreads) {
    acc = fmaf(xr[k] * sr[k / gs], static_cast<float>(wr[k]), acc);
  }
#pragma unroll
  for (int off = 32; off >= 1; off /= 2) acc += __shfl_xor(acc, off, kWave);
  if ((tid & (kWave - 1)) == 0) red[tid >> 6] = acc;
  __syncthreads();
  if (tid == 0) {
    float v = red[0];
#pragma unroll
    for (int wv = 1; wv < kWaves; ++wv) v += red[wv];
    y[static_cast<size_t>(m) * N + n] = v;
  }
}

template <int R, int MT>
hipError_t launch_rows(const float* x, const int8_t* w, const float* s, float* y, int M, int N,
                       int K, int gs, hipStream_t st) {
  const dim3 grid((N + R - 1) / R);
  if (gs == 64) {
    hipLaunchKernelGGL((gemv_rows_kernel<R, MT, 64>), grid, dim3(kThreads), 0, st, x, w, s, y, M,
                       N, K, gs);
  } else {
    hipLaunchKernelGGL((gemv_rows_kernel<R, MT, 0>), grid, dim3(kThreads), 0, st, x, w, s, y, M,
                       N, K, gs);
  }
  return hipGetLastError();
}

}  // namespace

int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

namespace {

// Launch configurations measured best on MI355X (Llama-3-8B and Qwen2-1.5B decode steps; the
// values are macros so that variants can be built for A/B runs without editing the dispatch):
//   NORM_WV         waves per workgroup of the RMSNorm-prologue GEMV with rows of 2-8 KiB (each
//                   workgroup re-stages the normalised row: fewer, larger workgroups stage it
//                   fewer times);
//   NARROW_WPC      resident waves per CU for N <= 8192 (12, 24 and 32 measured slower);
//   PAIR_WV, _WPC   the row-pair (gate/up + SwiGLU) GEMV: 8-wave workgroups, 16 waves per CU
//                   (4-wave: 22.6 -> 23.7 us on Llama gate/up; 7 waves: 35 us; 24-32 per CU slower);
//   PAIR_U1536      1 KiB steps per row for 1024 < K <= 2048 when 1: 2 (one masked 2 KiB step
//                   for K = 1536) measured faster;
//   SPLITROW_*      two waves per row (U chunks of 1 KiB each) in 16-wave workgroups for the plain
//                   few-long-rows shape (Qwen2 down: 1122 against 1056 tokens/s unsplit; 3 or 4
//                   waves per row, 8- or 15-wave workgroups, one wave of 9 chunks all slower).
#ifndef SQ8_GEMV_NORM_WV
#define SQ8_GEMV_NORM_WV 8
#endif
#ifndef SQ8_GEMV_NARROW_WPC
#define SQ8_GEMV_NARROW_WPC 16
#endif
#ifndef SQ8_GEMV_PAIR_WV
#define SQ8_GEMV_PAIR_WV 8
#endif
#ifndef SQ8_GEMV_PAIR_WPC
#define SQ8_GEMV_PAIR_WPC 16
#endif
#ifndef SQ8_GEMV_PAIR_U1536
#define SQ8_GEMV_PAIR_U1536 2
#endif
#ifndef SQ8_GEMV_SPLITROW_WV
#define SQ8_GEMV_SPLITROW_WV 16
#endif
#ifndef SQ8_GEMV_SPLITROW_U
#define SQ8_GEMV_SPLITROW_U 5
#endif
#ifndef SQ8_GEMV_SPLITROW_KS
#define SQ8_GEMV_SPLITROW_KS 2
#endif

// LDS bytes the stream kernel may use for staged token rows (MT * K fp32).
constexpr size_t kStreamLdsMax = 64 * 1024;
// Two token rows of long K (down projections) may stage up to 128 KiB: fewer workgroups per CU,
// but the sweep still streams at the single-row rate, against half that for the rows kernel.
constexpr size_t kStreamLdsTwoRows = 128 * 1024;

// WV waves per workgroup; 16 waves per CU in total, fewer when there are fewer row blocks.
template <int R, int U, int MT, int GS, int WV, int PRO, bool PAIR>
hipError_t launch_sweep_t(const float* x, const int8_t* w, const float* s, float* y, int M, int N,
                          int K, int gs, const ProArgs& pro, hipStream_t st, int wpc) {
  const size_t lds = static_cast<size_t>(MT) * K * sizeof(float);
  const int nblk = (N + R - 1) / R;
  const int grid = min((nblk + WV - 1) / WV, (wpc / WV) * cu_count());
  if (lds > 64 * 1024) {  // above 64 KiB the dynamic LDS size needs the opt-in attribute
    static std::atomic<uint64_t> done_full{0}, done_tail{0};
    hipError_t e = ensure_dynamic_lds(
        reinterpret_cast<const void*>(sweep_kernel<R, U, MT, GS, false, WV, PRO, PAIR>),
        kStreamLdsTwoRows, done_full);
    if (e == hipSuccess)
      e = ensure_dynamic_lds(
          reinterpret_cast<const void*>(sweep_kernel<R, U, MT, GS, true, WV, PRO, PAIR>),
          kStreamLdsTwoRows, done_tail);
    if (e != hipSuccess) return e;
  }
  if (K % (1024 * U) == 0) {
    hipLaunchKernelGGL((sweep_kernel<R, U, MT, GS, false, WV, PRO, PAIR>), dim3(grid), dim3(WV * kWave),
                       lds, st, x, w, s, y, M, N, K, gs, pro);
  } else {
    hipLaunchKernelGGL((sweep_kernel<R, U, MT, GS, true, WV, PRO, PAIR>), dim3(grid), dim3(WV * kWave),
                       lds, st, x, w, s, y, M, N, K, gs, pro);
  }
  return hipGetLastError();
}

// wpc: resident waves per CU the grid is sized for.
template <int R, int U, int WV, int MT, int PRO = kProNone, bool PAIR = false>
hipError_t launch_sweep(const float* x, const int8_t* w, const float* s, float* y, int M, int N,
                        int K, int gs, hipStream_t st, const ProArgs& pro = {}, int wpc = 16) {
  return gs == 64
             ? launch_sweep_t<R, U, MT, 64, WV, PRO, PAIR>(x, w, s, y, M, N, K, gs, pro, st, wpc)
             : launch_sweep_t<R, U, MT, 0, WV, PRO, PAIR>(x, w, s, y, M, N, K, gs, pro, st, wpc);
}

// Configurations measured best on the Llama-3-8B and Qwen2-1.5B shapes. Rows of 8 KiB and more:
// one row per wave; 7 KiB steps in 16-wave workgroups when K is a multiple of 7 KiB (Llama down,
// 14 KiB rows), else 4 KiB steps in 8-wave workgroups (Qwen2 down, 8.75 KiB rows). Shorter rows:
// a step covers the row in at most 4 iterations of 1 KiB, so short rows (1.5 KiB) do not issue
// masked loads; up to 8192 rows one row per wave in 8-wave workgroups, more rows 2 rows per wave
// in 4-wave workgroups.
// Split-row GEMV (M = 1): KS waves per row, U chunks of 1 KiB per wave, WV waves per workgroup.
template <int U, int KS, int WV, int PRO>
hipError_t launch_splitrow(const float* x, const int8_t* w, const float* s, float* y, int N, int K,
                           int gs, hipStream_t st, const ProArgs& pro) {
  const size_t lds = static_cast<size_t>(K) * sizeof(float);
  const dim3 grid((N + WV / KS - 1) / (WV / KS));
  const bool tail = K != KS * U * 1024;
  if (gs == 64) {
    if (tail)
      hipLaunchKernelGGL((splitrow_kernel<U, KS, WV, 64, true, PRO>), grid, dim3(WV * kWave), lds,
                         st, x, w, s, y, N, K, gs, pro);
    else
      hipLaunchKernelGGL((splitrow_kernel<U, KS, WV, 64, false, PRO>), grid, dim3(WV * kWave), lds,
                         st, x, w, s, y, N, K, gs, pro);
  } else {
    hipLaunchKernelGGL((splitrow_kernel<U, KS, WV, 0, true, PRO>), grid, dim3(WV * kWave), lds, st,
                       x, w, s, y, N, K, gs, pro);
  }
  return hipGetLastError();
}

template <int MT, int PRO = kProNone>
hipError_t launch_stream(const float* x, const int8_t* w, const float* s, float* y, int M, int N,
                         int K, int gs, hipStream_t st, const ProArgs& pro = {}) {
  // Few long rows behind a fused prologue (Qwen2-1.5B down projection: 1536 rows of 8.75 KiB):
  // two waves per row, 8 rows per 16-wave workgroup. The prologue is recomputed by every
  // workgroup, so the workgroup count stays that of one row per wave in 8-wave workgroups (with
  // 8-wave split-row workgroups, twice as many, the decode step measured slower).
  if (MT == 1 && PRO != kProNone && N <= 2048 && K >= 8192 && K <= 10 * 1024)
    return launch_splitrow<5, 2, 16, PRO>(x, w, s, y, N, K, gs, st, pro);
  // The same few long rows without a prologue (Qwen2-1.5B down projection behind the SwiGLU
  // epilogue of gate/up): two waves per row, SQ8_GEMV_SPLITROW_WV waves per workgroup.
#if SQ8_GEMV_SPLITROW_WV > 0
  if (MT == 1 && PRO == kProNone && N <= 2048 && K >= 8192 && K <= 10 * 1024)
    return launch_splitrow<SQ8_GEMV_SPLITROW_U, SQ8_GEMV_SPLITROW_KS, SQ8_GEMV_SPLITROW_WV, PRO>(
        x, w, s, y, N, K, gs, st, pro);
#endif
  if (K >= 8192) {
    return K % 7168 == 0 ? launch_sweep<1, 7, 16, MT, PRO>(x, w, s, y, M, N, K, gs, st, pro)
                         : launch_sweep<1, 4, 8, MT, PRO>(x, w, s, y, M, N, K, gs, st, pro);
  }
  const int u = K <= 1024 ? 1 : (K <= 2048 ? 2 : 4);
  if (N <= 8192) {
    const int wpc = SQ8_GEMV_NARROW_WPC;
    if (u == 1) return launch_sweep<1, 1, 8, MT, PRO>(x, w, s, y, M, N, K, gs, st, pro, wpc);
    if (u == 2) return launch_sweep<1, 2, 8, MT, PRO>(x, w, s, y, M, N, K, gs, st, pro, wpc);
    if (PRO == kProNorm)  // every workgroup recomputes the norm: workgroup size is a lab knob
      return launch_sweep<1, 4, SQ8_GEMV_NORM_WV, MT, PRO>(x, w, s, y, M, N, K, gs, st, pro, wpc);
    return launch_sweep<1, 4, 8, MT, PRO>(x, w, s, y, M, N, K, gs, st, pro, wpc);
  }
  if (u == 1) return launch_sweep<2, 1, 4, MT, PRO>(x, w, s, y, M, N, K, gs, st, pro);
  if (u == 2) return launch_sweep<2, 2, 4, MT, PRO>(x, w, s, y, M, N, K, gs, st, pro);
  if (PRO == kProNone && MT == 1) {
    // One row per wave when that spreads the row blocks more evenly over the 16 waves per CU
    // (Llama gate/up: 28672 rows = exactly 7 per wave, against 3.5 two-row blocks: +1 % on the
    // decode step).
    const double waves = 16.0 * cu_count();
    const double b1 = N / waves, b2 = N / (2.0 * waves);
    if (b1 / std::ceil(b1) > b2 / std::ceil(b2) + 0.01)
      return launch_sweep<1, 4, 8, MT, PRO>(x, w, s, y, M, N, K, gs, st, pro);
  }
  return launch_sweep<2, 4, 4, MT, PRO>(x, w, s, y, M, N, K, gs, st, pro);
}

}  // namespace

// Token rows are staged padded to 1, 2 or 4.
bool gemv_stream_fits(int M, int K) {
  const int mt = M <= 1 ? 1 : (M <= 2 ? 2 : 4);
  const size_t cap = mt == 2 ? kStreamLdsTwoRows : kStreamLdsMax;
  return M <= 4 && static_cast<size_t>(mt) * K * sizeof(float) <= cap;
}

// Requires: group_size % 16 == 0, K % group_size == 0, 16-byte aligned x and w.
hipError_t launch_gemv(const float* x, const int8_t* w, const float* s, float* y, int M, int N,
                       int K, int gs, hipStream_t st) {
  if (gemv_stream_fits(M, K)) {
    if (M == 1) return launch_stream<1>(x, w, s, y, M, N, K, gs, st);
    if (M == 2) return launch_stream<2>(x, w, s, y, M, N, K, gs, st);
    return launch_sweep<1, 4, 8, 4>(x, w, s, y, M, N, K, gs, st);  // K <= 4096 here
  }
  if (M == 1) return launch_rows<8, 1>(x, w, s, y, M, N, K, gs, st);
  if (M == 2) return launch_rows<8, 2>(x, w, s, y, M, N, K, gs, st);
  return launch_rows<8, 4>(x, w, s, y, M, N, K, gs, st);
}

hipError_t launch_generic(const float* x, const int8_t* w, const float* s, float* y, int M, int N,
                          int K, int gs, hipStream_t st) {
  // One workgroup per (row, token); grid.y is limited to 65535 token rows per launch.
  for (int m0 = 0; m0 < M; m0 += 65535) {
    const int mc = min(M - m0, 65535);
    hipLaunchKernelGGL(generic_kernel, dim3(N, mc), dim3(kThreads), 0, st,
                       x + static_cast<size_t>(m0) * K, w, s, y + static_cast<size_t>(m0) * N,
                       mc, N, K, gs);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// Decode GEMV with a fused prologue (M = 1); the caller has validated the shape.
hipError_t launch_gemv_norm(const float* x, const float* res, float* x_out, const float* nw,
                            float eps, const int8_t* w, const float* s, float* y, int N, int K,
                            int gs, hipStream_t st) {
  const ProArgs pro{res, x_out, nw, eps};
  return launch_stream<1, kProNorm>(x, w, s, y, 1, N, K, gs, st, pro);
}

hipError_t launch_gemv_norm_swiglu(const float* x, const float* res, float* x_out,
                                  const float* nw, float eps, const int8_t* w, const float* s,
                                  float* y, int N, int K, int gs, hipStream_t st) {
  // Row pairs (gate b, up b + N/2) in two-row blocks, 4-wave workgroups, steps of up to 4 KiB
  // per row: the configuration of the plain wide-output GEMV with two rows per wave.
  const ProArgs pro{res, x_out, nw, eps};
  constexpr int WV = SQ8_GEMV_PAIR_WV;
  const int wpc = SQ8_GEMV_PAIR_WPC;
  if (K <= 1024)
    return launch_sweep<2, 1, WV, 1, kProNorm, true>(x, w, s, y, 1, N, K, gs, st, pro, wpc);
  if (K <= 2048 && (SQ8_GEMV_PAIR_U1536 == 2 || K % 1024 == 0))
    return launch_sweep<2, 2, WV, 1, kProNorm, true>(x, w, s, y, 1, N, K, gs, st, pro, wpc);
  if (K <= 2048)
    return launch_sweep<2, 1, WV, 1, kProNorm, true>(x, w, s, y, 1, N, K, gs, st, pro, wpc);
  return launch_sweep<2, 4, WV, 1, kProNorm, true>(x, w, s, y, 1, N, K, gs, st, pro, wpc);
}

hipError_t launch_gemv_swiglu(const float* ab, const int8_t* w, const float* s, float* y, int N,
                              int K, int gs, hipStream_t st) {
  return launch_stream<1, kProSwiGLU>(ab, w, s, y, 1, N, K, gs, st);
}

}  // namespace sq8
