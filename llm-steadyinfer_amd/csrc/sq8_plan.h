// Launch plans and address arithmetic of the MFMA and packed-GEMV kernels (sq8_mfma.hip).
//
// Everything here is plain C++ with no HIP dependency: the index functions are constexpr, which
// makes them callable from device code, and the plans take the CU count as an argument. The
// kernels and launchers call exactly these functions, and the CPU replay test compiles this same
// header with g++ and walks every weight, scale, activation, partial and ticket address each
// launch would touch, for the shapes the model stacks run (tests/cpp/test_index_replay.cpp).
#pragma once
#include <stddef.h>
#include <stdint.h>

#include <algorithm>

namespace sq8 {

constexpr int kWave = 64;  // CDNA wavefront width
constexpr int BK = 64;     // K per main-loop step = one weight group of 64

// Bytes of split-K tickets at the start of every MFMA workspace. They must be zero before the
// first call and every call leaves them zero, so no other use of a workspace may write there.
constexpr int kWsTicketBytes = 64 * 1024;
constexpr int kTicketBytes = kWsTicketBytes;

// K groups per split of the tile kernel: bounds its LDS scale stage (16*T rows x this many).
constexpr int kTileScaleGroups = 128;
// Decode GEMM configuration: 8 waves x 2 column tiles of 16, an 8-deep weight ring.
constexpr int kDgT = 2, kDgW = 8, kDgDepth = 8;
// Ring depth for RT row tiles: 4 tiles take 16 KiB of LDS per group, so their ring is shorter.
constexpr int dg_depth(int rt) { return rt >= 3 ? 4 : kDgDepth; }
constexpr int kDgCols = 16 * kDgT * kDgW;
// Groups per split at most: the LDS scale stage holds 256 columns x (64 + 1) floats. At 32 the
// 64-row Llama LM head (128256 x 4096) was split in two: 290 against 242 us unsplit.
constexpr int kDgScaleGroups = 64;
// Largest M served by the single-launch skinny kernel.
constexpr int kSkinnyMaxM = 32;
// Waves per workgroup of the packed GEMV.
constexpr int kPgWaves = 8;

#ifndef SQ8_PGEMV_U
#define SQ8_PGEMV_U 4
#endif
#ifndef SQ8_PGEMV_WPC
#define SQ8_PGEMV_WPC 2
#endif
#ifndef SQ8_PGEMV_MAX_M
#define SQ8_PGEMV_MAX_M 2
#endif
#ifndef SQ8_GEMM_GM
#define SQ8_GEMM_GM 4
#endif
// Token rows up to which packed weights take the GEMV (above, the int8-limb MFMA kernel).
constexpr int kPgMaxM = SQ8_PGEMV_MAX_M;

namespace ix {

constexpr int imin(int a, int b) { return a < b ? a : b; }

// Byte offset of a lane's 16 weights of group 0 of weight row `row`. A lane of a kernel that
// feeds v_mfma_f32_16x16x32_f16 (or the int8 MFMA) its B operand straight from memory takes, per
// 64-wide group g, the 16 bytes k = 64 g + 16 (lane / 16) .. +15 of weight row n
// (n % 16 == lane % 16). Row-major weights ([N][K], the reference's layout) hold them at
// n K + 64 g + 16 (lane / 16): a wave instruction covers 16 rows x 64 B. Packed weights
// (sq8_pack_weights) store each 16-row tile's group as one 1 KiB block in lane order,
// tile-major: the same 16 bytes sit at (n / 16) 16 K + 1024 g + 16 (16 (lane / 16) + n % 16),
// so a wave instruction reads 1 KiB contiguously and a tile's K range is one run of 16 K bytes.
// The packed address uses the row's own place in its tile, row % 16, so rows whose place
// differs from the lane's, such as the up rows of a fused gate/up weight with N / 2 % 16 != 0,
// are read correctly.
constexpr size_t lane_woff(int pk, int row, int K, int lane) {
  return pk ? static_cast<size_t>(row >> 4) * K * 16 +
                  static_cast<size_t>(((lane >> 4) * 16 + (row & 15)) * 16)
            : static_cast<size_t>(row) * K + (lane >> 4) * 16;
}
// Byte distance between consecutive 64-wide groups of one lane's weights.
constexpr int wgroup_step(int pk) { return pk ? 1024 : 64; }
// Bytes of a packed weight buffer: whole 16-row tiles, zero rows past N.
constexpr size_t packed_bytes(int N, int K) { return static_cast<size_t>((N + 15) / 16) * 16 * K; }

// Weight row (output column) of each MFMA kernel's lane. Skinny kernels: wave `wave`'s column
// tile j of the workgroup starting at column n0.
constexpr int skinny_row(int n0, int wave, int TN, int j, int lcol, int N) {
  return imin(n0 + (wave * TN + j) * 16 + lcol, N - 1);
}
// Tile kernel: column tile j of the workgroup starting at column n0 (every wave of the workgroup
// reads the same T tiles over different K groups).
constexpr int tile_row(int n0, int j, int lcol, int N) { return imin(n0 + 16 * j + lcol, N - 1); }
// Decode GEMM: workgroup column c = (wave T + j) 16 + l of workgroup bx (COLS = 16 T W columns).
// SwiGLU (N = 2F rows [gate; up]): tiles j < T/2 of a wave hold the gate rows of the wave's
// features, tiles j >= T/2 the matching up rows.
constexpr int dgemm_row(int c, int bx, int T, int W, int N, bool swiglu) {
  const int COLS = 16 * T * W, HT = T / 2;
  if (!swiglu) return imin(bx * COLS + c, N - 1);
  const int F = N / 2, f0 = bx * (COLS / 2);
  const int wv = c / (16 * T), j = (c / 16) % T, l = c % 16;
  const int f = f0 + (wv * HT + j % HT) * 16 + l;
  return imin(f, F - 1) + (j >= HT ? F : 0);
}
// Prefill GEMM: tile column c (0 <= c < BN) of workgroup column bx; each wave owns TN 32-column
// tiles. SwiGLU: the workgroup owns features f0 .. f0 + BN/2 - 1 of F = N/2; a wave's tiles
// j < TN/2 hold the gate rows of its features and tiles j + TN/2 their up rows (F rows on).
constexpr int gemm_feat(int c, int bx, int BN, int TN) {  // SwiGLU feature of tile column c
  const int HT = TN / 2, f0 = bx * (BN / 2);
  const int tl = c >> 5, jj = (tl % TN) % HT;
  return f0 + ((tl / TN) * HT + jj) * 32 + (c & 31);
}
constexpr int gemm_row(int c, int bx, int BN, int TN, int N, bool swiglu) {
  if (!swiglu) return imin(bx * BN + c, N - 1);
  const int F = N / 2;
  return imin(gemm_feat(c, bx, BN, TN), F - 1) + (((c >> 5) % TN) >= TN / 2 ? F : 0);
}
// Prefill GEMM: byte offset, relative to the stage's weight base, of 16-byte chunk q of weight
// row n in one K stage (q / 4: the stage's group, q % 4: its 16-byte piece). The stage base
// advances by stage_wstep per stage.
constexpr uint32_t gemm_woff(int pk, uint32_t n, int K, int q) {
  return pk ? (n >> 4) * static_cast<uint32_t>(K) * 16u + (q >> 2) * 1024u +
                  ((q & 3) * 16u + (n & 15u)) * 16u
            : n * static_cast<uint32_t>(K) + q * 16u;
}
constexpr size_t gemm_stage_wstep(int pk, int GPS) {
  return pk ? static_cast<size_t>(GPS) * 1024 : static_cast<size_t>(GPS) * BK;
}

// Output tile of the prefill GEMM's hardware workgroup (bx, by, bz) in a grid X x Y x Z.
// MI355X hands workgroups to its 8 XCDs round robin (workgroup b runs on XCD b % 8), and each XCD
// has its own L2. The grid is renumbered so that each XCD works through one contiguous range of
// tiles, ordered in bands of GM M-tiles (column by column within a band): the ~32 workgroups an
// XCD runs at once then share GM activation tiles and 32 / GM weight tiles in its L2. A
// bijection when the grid is a multiple of 8 workgroups; otherwise, and for a single M-tile,
// the launch order is kept.
struct Tile3 {
  int x, y, z;
};
constexpr Tile3 gemm_tile(int bx, int by, int bz, int X, int Y, int Z, int GM) {
  const int total = X * Y * Z;
  if (GM <= 0 || Y == 1 || total % 8 != 0) return Tile3{bx, by, bz};
  const int b = bx + X * (by + Y * bz);
  const int L = (b & 7) * (total >> 3) + (b >> 3);
  const int XY = X * Y;
  const int z = L / XY;
  const int r = L - z * XY;
  const int band = r / (GM * X), row0 = band * GM;
  const int rows = imin(GM, Y - row0);
  const int q = r - band * GM * X;
  return Tile3{q / rows, row0 + q % rows, z};
}

// Packed GEMV. Unit u = (tile, slice): 16 weight rows and the KS groups g0 .. g0 + gn - 1.
// Weight read of step slot i (0 <= i < gn) by lane `lane`: 16 bytes at pg_wbase + 1024 i.
constexpr size_t pg_wbase(int tile, int K, int g0, int lane) {
  return static_cast<size_t>(tile) * K * 16 + static_cast<size_t>(g0) * 1024 +
         static_cast<size_t>(lane) * 16;
}
// Group slot the step's load v reads: slots past the slice re-read its last group (their scale
// is 0), so each step issues U loads unconditionally.
constexpr int pg_wslot(int i0, int v, int gn) { return imin(i0 + v, gn - 1); }
// Scale float4 of step loads v .. v + 3: with gn % 4 == 0 the last whole float4 of the slice is
// gn - 4; slots past gn read it again and get scale 0.
constexpr int pg_sslot(int i0, int v, int gn) { return imin(i0 + v, gn - 4); }
// First scale (in floats) of the lane's row in the slice; rows past N read row N - 1.
constexpr size_t pg_srow(int tile, int lcol, int N, int G, int g0) {
  return static_cast<size_t>(imin(tile * 16 + lcol, N - 1)) * G + g0;
}
// Partial sum (in floats) of slice sl, token row m, output n.
constexpr size_t pg_part(int sl, int M, int m, int N, int n) {
  return (static_cast<size_t>(sl) * M + m) * N + n;
}
// Source (in floats) of LDS float4 c of the staged activations (MT rows; rows past M repeat M-1).
constexpr size_t pg_xsrc(int c, int K4, int M, int K) {
  return static_cast<size_t>(imin(c / K4, M - 1)) * K + 4 * static_cast<size_t>(c % K4);
}

// Decode GEMV (sweep_kernel, splitrow_kernel in sq8_gemv.hip): these restate the kernels'
// expressions for the CPU replay. The kernels keep their own spelling of the same arithmetic
// (block_row, the step's k and kc, the stage swizzle), which compiles to the code that was
// measured; routed through these functions, hipcc schedules the sweep differently.
// A row block b holds R consecutive weight rows, or with `pair` (R = 2, a fused [gate; up] weight
// of N = 2F rows) gate row b and its up row b + F; rows past N (blocks past the last) read row
// N - 1 and their sums are dropped.
constexpr int sw_nblk(int N, int R, bool pair) { return pair ? N / 2 : (N + R - 1) / R; }
constexpr int sw_row(int b, int r, int R, int N, bool pair) {
  return pair ? imin(b + r * (N / 2), N - 1) : imin(b * R + r, N - 1);
}
// First K byte of lane `lane`'s 16 weights in 1 KiB chunk c of a row (c = st U + u for step st
// of U chunks); with `tail` (K not a multiple of the step), chunks past K read the row's first
// 16 bytes and are dropped.
constexpr int sw_k(int c, int lane) { return c * 1024 + lane * 16; }
constexpr int sw_kc(int k, int K, bool tail) { return !tail || k < K ? k : 0; }
// LDS slot of staged float4 number i (bank-conflict swizzle inside each aligned group of 4
// float4, so a lane's 4 float4 of a 16-element chunk stay in the group).
constexpr int sw_xslot(int i) { return i ^ ((i >> 4) & 3); }

// Prefill GEMM LDS swizzles (GPS groups per stage: x rows of 8 GPS 16-byte chunks, w rows of
// 4 GPS): x row r keeps chunk c at slot c ^ swz_x(r), w row r keeps chunk q at slot q ^ swz_w(r).
template <int GPS>
constexpr int swz_x(int r) {
  return GPS == 1 ? (r ^ (r >> 3)) & 7 : r & 15;
}
template <int GPS>
constexpr int swz_w(int r) {
  return GPS == 1 ? ((r >> 1) ^ (r >> 2)) & 3 : (r ^ (r >> 3)) & 7;
}

}  // namespace ix

// Prefill GEMM tile: WAVES_M x WAVES_N waves, each TM x TN tiles of 32 x 32, STAGES LDS stages of
// GPS groups each.
template <int WAVES_M, int WAVES_N, int TM, int TN, int STAGES, int GPS>
struct PTile {
  static constexpr int NW = WAVES_M * WAVES_N;
  static constexpr int NT = NW * kWave;
  static constexpr int BM = WAVES_M * TM * 32;
  static constexpr int BN = WAVES_N * TN * 32;
  static constexpr int KB = BK * GPS;            // K per stage
  static constexpr int CX = 8 * GPS;             // 16-byte chunks per staged x row (hi or lo)
  static constexpr int CW = 4 * GPS;             // 16-byte chunks per staged weight row
  static constexpr int XB = BM * CX * 16;        // bytes of x hi (or lo) per stage
  static constexpr int WB = BN * CW * 16;        // bytes of int8 weights per stage
  static constexpr int SB = GPS * BN * 8;        // scale bytes per stage (each 32-column run twice)
  static constexpr int STAGE = 2 * XB + WB + SB;
  static constexpr size_t LDS_BYTES = static_cast<size_t>(STAGES) * STAGE;
  static constexpr int XL = BM * CX / NT;        // x DMA instructions per thread per stage (hi or lo)
  static constexpr int WL = BN * CW / NT;        // weight DMA instructions per thread per stage
  static constexpr int SL = GPS * BN / 32 / NW;  // scale DMA instructions per thread per stage
  static constexpr int LOADS = 2 * XL + WL + SL;
  static_assert(XL >= 1 && WL >= 1 && SL >= 1 && BM * CX % NT == 0 && BN * CW % NT == 0 &&
                    (GPS * BN / 32) % NW == 0,
                "tile does not match the DMA pattern");
  static_assert((STAGES - 2) * LOADS < 64, "vmcnt range");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
};


// ---------------------------------------------------------------- MFMA path plans
struct Plan {
  bool tile;      // pack_x_kernel + tile_kernel (9 <= M <= 64)
  bool dgemm;     // pack_x_kernel + dgemm_kernel (+ splitk_reduce_kernel); uses rt
  int rt, tn, tw; // tile: 16-row activation tiles, 16-column tiles per wave, waves per workgroup
  bool skinny;
  int kw;         // skinny: K groups per chunk (divides groups_per_split)
  int cfg;        // GEMM: 1: 64x256 tile, 2: 128x256.  Skinny: 0: MT=1, 1: MT=2
  int gps;        // GEMM: 64-wide groups per K stage (the split is counted in stages)
  int bm, bn;
  int splits;
  int groups_per_split;
};

// Plan for M token rows on a GPU of `cus` compute units.
inline Plan make_plan_for(int M, int N, int K, int cus) {
  Plan p{};
  const int nsteps = K / BK;
  const int target = 2 * cus;
  const int rt = (M + 15) / 16;
  // Tile kernel for 9..64 tokens, except long rows (K >= 8192) at 16 or fewer tokens (the skinny
  // kernel is faster there) and at more than 32 tokens (the GEMM is). Configurations from MI355X
  // sweeps over the Llama-3-8B projections: wide outputs (N >= 16384) take 4 column tiles per
  // wave and no K split; others take 2 tiles, 8 waves, and split K when the grid has at most
  // 1024 waves.
  // Decode GEMM for wide outputs at 33-64 tokens (Llama gate/up at 48 and 64 rows: 59 and 63 us
  // against 70 and 77 for the tile kernel, which stays ahead on narrower outputs, where the
  // decode GEMM needs a deep K split to fill the GPU).
  // 17-32 tokens on wide outputs up to 64Ki columns take it too (Llama gate/up at 24 and 32
  // rows: 53.4 and 53.7 us against 56.6 and 56.3; the 128256-column LM head stays on the tile
  // kernel, 209 against 217 us at 24 rows, as do 16 or fewer rows, 47.5 against 50.2).
  if (M <= 64 && N >= 16384 && (M > 32 || (M > 16 && N <= 65536))) {
    p.dgemm = true;
    p.rt = rt;
    const int tiles = (N + kDgCols - 1) / kDgCols;
    const int want = std::max(1, (cus + tiles / 2) / tiles);
    int gpsplit = (nsteps + want - 1) / want;
    gpsplit = (gpsplit + kDgDepth - 1) / kDgDepth * kDgDepth;
    p.groups_per_split = std::min(std::min(gpsplit, nsteps), kDgScaleGroups);
    p.splits = (nsteps + p.groups_per_split - 1) / p.groups_per_split;
    return p;
  }
  if (M > 8 && M <= 64 && !(K >= 8192 && (rt == 1 || rt > 2))) {
    p.tile = true;
    p.rt = rt;
    int splits = 1;
    if (N >= 16384) {
      p.tn = 4;
      p.tw = rt <= 2 ? 4 : 2;
    } else {
      p.tn = 2;
      p.tw = 8;
      const int waves = ((N + 31) / 32) * p.tw;
      const int smax = std::max(1, nsteps / p.tw);  // at least one group per wave
      if (waves <= 1024) splits = std::min(smax, (2048 + waves - 1) / waves);
    }
    splits = std::max(splits, (nsteps + kTileScaleGroups - 1) / kTileScaleGroups);
    p.groups_per_split = (nsteps + splits - 1) / splits;
    p.splits = (nsteps + p.groups_per_split - 1) / p.groups_per_split;
    return p;
  }
  if (M <= kSkinnyMaxM) {
    p.skinny = true;
    p.cfg = 0;
    p.bm = M <= 8 ? 8 : ((M + 15) / 16) * 16;
    p.bn = 64;
    const int blocks = (N + p.bn - 1) / p.bn;
    const int kw_max = M <= 32 ? 4 : 2;
    p.kw = 1;
    while (p.kw < kw_max && nsteps % (2 * p.kw) == 0) p.kw *= 2;
    const int chunks = nsteps / p.kw;
    int splits = 1;
    if (blocks < target && blocks <= kTicketBytes / 4)
      splits = std::min(chunks, (target + blocks - 1) / blocks);
    const int cps = (chunks + splits - 1) / splits;  // chunks per split
    p.groups_per_split = cps * p.kw;
    p.splits = (chunks + cps - 1) / cps;
    return p;
  }
  // Pipelined GEMM: one 64 x 256 (M <= 64; 2 stages of 2 groups, 136 KiB of LDS, or 3 stages
  // of one group when K is an odd number of groups) or 128 x 256 tile (3 stages of one group,
  // 150 KiB) per workgroup, one workgroup per CU. K is split when that evens out the rounds of
  // workgroups over the CUs: cost = rounds / splits plus a small charge per split for the
  // partial tiles and the reduction.
  p.cfg = M <= 64 ? 1 : 2;
  // 64-row tiles stream weights: two groups per stage read each weight row 128 bytes (one L2
  // line) at a time (Llama down projection at 64 rows: 46 against 51 us with one group).
  p.gps = p.cfg == 1 && K % (2 * BK) == 0 ? 2 : 1;
  const int nst = nsteps / p.gps;
  p.bm = M <= 64 ? 64 : 128;
  p.bn = 256;
  const int tiles = ((M + p.bm - 1) / p.bm) * ((N + p.bn - 1) / p.bn);
  int splits = 1;
  double best = 1e30;
  // The 64-row tile streams weights (partials are cheap next to them); the 128-row tile is
  // MFMA-bound and pays more for its partials.
  const double charge = p.cfg == 1 ? 0.005 : 0.04;
  for (int sp = 1; sp <= 16 && sp * 4 <= nsteps; ++sp) {
    const double rounds = static_cast<double>((tiles * sp + cus - 1) / cus);
    const double cost = rounds / sp + charge * (sp - 1);
    if (cost < best - 1e-9) { best = cost; splits = sp; }
  }
  p.groups_per_split = (nst + splits - 1) / splits;
  p.splits = (nst + p.groups_per_split - 1) / p.groups_per_split;
  return p;
}

// ---------------------------------------------------------------- packed GEMV plan
struct PgPlan {
  int ks, S, grid;
  size_t lds;
};
// ks groups per slice (a multiple of 4: whole float4s of scales), S slices per 16-row tile, and
// a grid of resident workgroups (wpc per CU when the staged activations leave room for them).
inline PgPlan pgemv_plan_for(int M, int N, int K, int cus, int wpc) {
  PgPlan p{};
  const int G = K / BK, ntiles = (N + 15) / 16;
  p.lds = static_cast<size_t>(M) * K * sizeof(float);
  const int wgs = p.lds > 80 * 1024 ? 1 : wpc;  // resident workgroups per CU
  p.grid = cus * wgs;
  const int slots = p.grid * kPgWaves;
  int S = std::max(1, (slots + ntiles - 1) / ntiles);
  if (ntiles > kTicketBytes / 4) S = 1;
  int ks = (G + S - 1) / S;
  ks = std::max(4, (ks + 3) / 4 * 4);  // whole float4s of scales
  p.ks = ks;
  p.S = (G + ks - 1) / ks;
  p.grid = std::min(p.grid, (ntiles * p.S + kPgWaves - 1) / kPgWaves);
  return p;
}

// Packed weights at 1-2 token rows with group size 64 and whole float4s of scales per row
// (s16: the scales are 16-byte aligned).
inline bool pgemv_ok_for(int M, int K, int gs, bool s16) {
  return M <= kPgMaxM && gs == BK && K % (4 * BK) == 0 && s16 &&
         static_cast<size_t>(M) * K * sizeof(float) <= 144 * 1024;
}

}  // namespace sq8
