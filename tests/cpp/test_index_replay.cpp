// CPU replay of the address arithmetic of the MFMA and packed-GEMV kernels.
//
// The kernels in llm-steadyinfer_amd/csrc/sq8_mfma.hip take their launch plans and every
// weight/scale/activation/partial index from sq8_plan.h. This program compiles that same header on
// the host and walks, lane by lane, every address a launch would touch for the shapes the model
// stacks run (Llama-3-8B and Qwen2-1.5B projections and LM heads, fused gate/up weights whose
// half is not a multiple of 16 rows, N = 1..64), and checks:
//  * every load lies inside its buffer and is aligned for its width;
//  * each weight load, decoded through the packed layout's own definition (the packing kernel:
//    16-byte unit d holds lane d % 64 of group (d / 64) % G of tile d / (64 G), i.e. row
//    16 tile + lane % 16, bytes 64 g + 16 (lane / 16) ..) or the row-major layout, is the weight
//    row and K range the lane multiplies;
//  * every (row < N, group, 16-byte quarter) is read exactly once per launch for its output, and
//    every scale a lane applies is that row's scale for that group;
//  * split-K partial and ticket indices stay in the workspace the library sizes;
//  * the prefill GEMM's XCD tile order is a bijection and its LDS swizzle loads each staged
//    chunk once.
// Two mutations of the index functions must be caught (the replay has teeth): the packed GEMV's
// scale read without its clamp at 8 groups per step (the over-read that faulted a lab build), and
// a packed weight address that takes the row's place in its tile from the lane instead of the row.
// Exit status 0 when every check passes.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "sq8_plan.h"

using namespace sq8;

namespace {

long g_fail = 0;
long g_checks = 0;
std::string g_ctx;
bool g_quiet = false;  // mutation runs count failures without printing them

void fail(const char* what, long long a, long long b) {
  ++g_fail;
  if (!g_quiet && g_fail <= 20) std::printf("FAIL [%s] %s (%lld, %lld)\n", g_ctx.c_str(), what, a, b);
}
#define CHECK(cond, what, a, b)                                  \
  do {                                                           \
    ++g_checks;                                                  \
    if (!(cond)) fail(what, (long long)(a), (long long)(b));     \
  } while (0)

struct Mut {
  bool scale_unclamped = false;  // pgemv: scale float4 at i0 + v instead of min(i0 + v, gn - 4)
  bool lane_place = false;       // packed address: row % 16 taken from lane % 16
};

size_t woff(const Mut& mu, int pk, int row, int K, int lane) {
  if (mu.lane_place && pk)
    return static_cast<size_t>(row >> 4) * K * 16 +
           static_cast<size_t>(((lane >> 4) * 16 + (lane & 15)) * 16);
  return ix::lane_woff(pk, row, K, lane);
}

// Weight row and first K index of the 16 bytes at byte offset `off` of a weight buffer.
struct RowK {
  long row, k;
};
RowK decode(int pk, size_t off, int K) {
  if (!pk) return RowK{static_cast<long>(off / K), static_cast<long>(off % K)};
  const int G = K / BK;
  const size_t d = off / 16;
  const long L = static_cast<long>(d % 64), g = static_cast<long>((d / 64) % G);
  const long t = static_cast<long>(d / (64 * static_cast<size_t>(G)));
  return RowK{16 * t + L % 16, 64 * g + 16 * (L / 16) + static_cast<long>(off % 16)};
}
size_t wbytes(int pk, int N, int K) {
  return pk ? ix::packed_bytes(N, K) : static_cast<size_t>(N) * K;
}
// One 16-byte weight load at `off` that must hold row `row`, K bytes k .. k + 15.
void check_wload(int pk, size_t off, int N, int K, long row, long k) {
  CHECK(off % 16 == 0, "weight load alignment", off, 16);
  CHECK(off + 16 <= wbytes(pk, N, K), "weight load past the buffer", off, wbytes(pk, N, K));
  const RowK rk = decode(pk, off, K);
  CHECK(rk.row == row, "weight load row", rk.row, row);
  CHECK(rk.k == k, "weight load k", rk.k, k);
}

// Coverage of (row, group, quarter) reads; each must be read once.
struct Cover {
  std::vector<unsigned char> c;
  int N, G;
  Cover(int n, int g) : c(static_cast<size_t>(n) * g * 4, 0), N(n), G(g) {}
  void hit(long row, long g, int q) {
    if (row < 0 || row >= N || g < 0 || g >= G) return;
    unsigned char& v = c[(static_cast<size_t>(row) * G + g) * 4 + q];
    if (v < 255) ++v;
  }
  void expect_once(const char* what) {
    long bad = 0, first = -1;
    for (size_t i = 0; i < c.size(); ++i)
      if (c[i] != 1) {
        if (first < 0) first = static_cast<long>(i);
        ++bad;
      }
    CHECK(bad == 0, what, bad, first);
  }
};

// ---------------------------------------------------------------- packed GEMV (1-2 rows)
void replay_pgemv(int M, int N, int K, int cus, int wpc, int U, const Mut& mu) {
  if (!pgemv_ok_for(M, K, BK, true)) return;
  const PgPlan p = pgemv_plan_for(M, N, K, cus, wpc);
  const int G = K / BK, ntiles = (N + 15) / 16, K4 = K / 4, MT = M;
  CHECK(p.ks % 4 == 0 && p.ks >= 4, "slice is whole float4s of scales", p.ks, 4);
  CHECK(static_cast<long>(p.S) * p.ks >= G && static_cast<long>(p.S - 1) * p.ks < G,
        "slices cover the groups", p.S, p.ks);
  CHECK(p.grid >= 1 && p.grid <= cus * wpc, "grid within the resident workgroups", p.grid, cus);
  CHECK(p.lds == static_cast<size_t>(MT) * K * 4 && p.lds <= 144 * 1024, "LDS", p.lds, 144 * 1024);
  if (p.S > 1) CHECK(ntiles <= kTicketBytes / 4, "tickets", ntiles, kTicketBytes / 4);
  // x staging into LDS
  for (int c = 0; c < MT * K4; ++c) {
    const size_t src = ix::pg_xsrc(c, K4, M, K);
    CHECK(src % 4 == 0 && src + 4 <= static_cast<size_t>(M) * K, "x staging read", src, M * K);
  }
  const size_t nscale = static_cast<size_t>(N) * G;
  const size_t nparts = static_cast<size_t>(p.S) * M * N;
  std::vector<unsigned char> pcov(p.S > 1 ? nparts : 0, 0);
  Cover cov(N, G);
  const long units = static_cast<long>(ntiles) * p.S;
  // Grid stride: unit u is taken by wave u % 8 of workgroup (u / 8) % grid; every u < units once.
  for (long u = 0; u < units; ++u) {
    const int tile = static_cast<int>(u / p.S), sl = static_cast<int>(u % p.S);
    const int g0 = sl * p.ks, gn = ix::imin(p.ks, G - g0);
    CHECK(gn >= 4 && gn % 4 == 0, "slice of whole float4s", gn, g0);
    for (int lane = 0; lane < 64; ++lane) {
      const int lcol = lane & 15, q = lane >> 4;
      const size_t wb = ix::pg_wbase(tile, K, g0, lane);
      const size_t sr = ix::pg_srow(tile, lcol, N, G, g0);
      const long row = 16L * tile + lcol;
      for (int i0 = 0; i0 < gn; i0 += U) {
        for (int v = 0; v < U; ++v) {
          const int slot = ix::pg_wslot(i0, v, gn);
          const size_t off = wb + static_cast<size_t>(slot) * 1024;
          // the packed buffer holds row 16 tile + lcol (a zero padding row past N)
          check_wload(1, off, N, K, row, 64L * (g0 + slot) + 16 * q);
          const int k4 = (g0 + slot) * 16 + q * 4;
          CHECK(k4 >= 0 && (MT - 1) * K4 + k4 + 4 <= MT * K4, "x LDS read", k4, K4);
          if (i0 + v < gn) cov.hit(row, g0 + i0 + v, q);
        }
        for (int v = 0; v < U; v += 4) {
          const int ss = mu.scale_unclamped ? i0 + v : ix::pg_sslot(i0, v, gn);
          const size_t at = sr + ss;
          CHECK(at % 4 == 0, "scale float4 alignment", at, 4);
          CHECK(at + 4 <= nscale, "scale float4 past the array", at, nscale);
          for (int t = 0; t < 4; ++t)
            if (i0 + v + t < gn) {
              const size_t want = static_cast<size_t>(ix::imin(static_cast<int>(row), N - 1)) * G +
                                  g0 + i0 + v + t;
              CHECK(at + t == want, "scale of the slot", at + t, want);
            }
        }
      }
      if (p.S > 1 && lane < 16 && row < N)
        for (int m = 0; m < M; ++m) {
          const size_t pi = ix::pg_part(sl, M, m, N, static_cast<int>(row));
          CHECK(pi < nparts, "partial index", pi, nparts);
          if (pi < nparts) ++pcov[pi];
        }
    }
  }
  cov.expect_once("packed GEMV reads each (row, group, quarter) once");
  for (size_t i = 0; i < pcov.size(); ++i)
    if (pcov[i] != 1) {
      CHECK(false, "partial written once", i, pcov[i]);
      break;
    }
}

// ---------------------------------------------------------------- skinny kernels (3-32 rows)
void replay_skinny(int M, int N, int K, int cus, int pk, const Mut& mu) {
  const Plan p = make_plan_for(M, N, K, cus);
  if (!p.skinny) return;
  const int G = K / BK, TN = 1, BN = 64 * TN, KW = p.kw;
  const int gx = (N + BN - 1) / BN;
  CHECK(KW == 1 || KW == 2 || KW == 4, "chunk width", KW, 0);
  CHECK(p.groups_per_split % KW == 0, "split of whole chunks", p.groups_per_split, KW);
  if (p.splits > 1) CHECK(gx <= kTicketBytes / 4, "tickets", gx, kTicketBytes / 4);
  const bool f4 = KW == 4 && G % 4 == 0;
  const size_t nscale = static_cast<size_t>(N) * G;
  Cover cov(N, G);
  for (int by = 0; by < p.splits; ++by) {
    const int gbeg = by * p.groups_per_split;
    const int gend = ix::imin(G, gbeg + p.groups_per_split);
    CHECK(gend > gbeg && (gend - gbeg) % KW == 0, "split holds whole chunks", gbeg, gend);
    const int nch = (gend - gbeg) / KW;
    // activation chunk reads (rows clamped to M - 1)
    const int MR = M <= 8 ? 8 : (M + 15) / 16 * 16;
    for (int f = 0; f < MR * KW * 16; ++f) {
      const int row = f / (KW * 16), rem = f % (KW * 16);
      for (int c = 0; c < nch; ++c) {
        const size_t at = static_cast<size_t>(ix::imin(row, M - 1)) * K +
                          static_cast<size_t>(gbeg + c * KW) * BK + rem * 4;
        CHECK(at + 4 <= static_cast<size_t>(M) * K, "x chunk read", at, M * K);
      }
    }
    for (int bx = 0; bx < gx; ++bx)
      for (int wave = 0; wave < 4; ++wave)
        for (int j = 0; j < TN; ++j)
          for (int lane = 0; lane < 64; ++lane) {
            const int lcol = lane & 15, q = lane >> 4;
            const int n0 = bx * BN;
            const int row = ix::skinny_row(n0, wave, TN, j, lcol, N);
            const size_t base =
                woff(mu, pk, row, K, lane) + static_cast<size_t>(gbeg) * ix::wgroup_step(pk);
            for (int c = 0; c < nch; ++c)
              for (int kk = 0; kk < KW; ++kk) {
                const int g = gbeg + c * KW + kk;
                check_wload(pk, base + static_cast<size_t>(c * KW + kk) * ix::wgroup_step(pk), N,
                            K, row, 64L * g + 16 * q);
                if (n0 + (wave * TN + j) * 16 + lcol < N) cov.hit(row, g, q);
              }
            for (int c = 0; c < nch; ++c) {
              const size_t s0 = static_cast<size_t>(row) * G + gbeg + c * KW;
              if (f4) CHECK(s0 % 4 == 0, "scale float4 alignment", s0, 4);
              CHECK(s0 + KW <= nscale, "scale read", s0, nscale);
            }
          }
  }
  cov.expect_once("skinny kernel reads each (row, group, quarter) once");
}

// ---------------------------------------------------------------- tile kernel (9-64 rows)
void replay_tile(int M, int N, int K, int cus, int pk, const Mut& mu) {
  const Plan p = make_plan_for(M, N, K, cus);
  if (!p.tile) return;
  const int G = K / BK, T = p.tn, W = p.tw;
  const int gx = (N + 16 * T - 1) / (16 * T);
  if (p.splits > 1) CHECK(gx <= kTicketBytes / 4, "tickets", gx, kTicketBytes / 4);
  Cover cov(N, G);
  const size_t nscale = static_cast<size_t>(N) * G;
  for (int by = 0; by < p.splits; ++by) {
    const int gsplit = by * p.groups_per_split;
    const int gcount = ix::imin(G, gsplit + p.groups_per_split) - gsplit;
    CHECK(gcount >= 1 && gcount <= kTileScaleGroups, "split within the scale stage", gcount,
          kTileScaleGroups);
    for (int bx = 0; bx < gx; ++bx) {
      const int n0 = bx * 16 * T;
      for (int r = 0; r < 16 * T; ++r)
        for (int gi = 0; gi < gcount; ++gi) {
          const size_t at = static_cast<size_t>(ix::imin(n0 + r, N - 1)) * G + gsplit + gi;
          CHECK(at < nscale, "scale stage read", at, nscale);
        }
      for (int wave = 0; wave < W; ++wave) {
        const int nst = wave < gcount ? (gcount - wave + W - 1) / W : 0;
        for (int j = 0; j < T; ++j)
          for (int lane = 0; lane < 64; ++lane) {
            const int lcol = lane & 15, q = lane >> 4;
            const int row = ix::tile_row(n0, j, lcol, N);
            const size_t base = woff(mu, pk, row, K, lane);
            for (int i = 0; i < nst; ++i) {
              const int g = gsplit + wave + i * W;
              CHECK(g < gsplit + gcount, "group inside the split", g, gsplit + gcount);
              check_wload(pk, base + static_cast<size_t>(g) * ix::wgroup_step(pk), N, K, row,
                          64L * g + 16 * q);
              if (n0 + 16 * j + lcol < N) cov.hit(row, g, q);
            }
          }
      }
    }
  }
  cov.expect_once("tile kernel reads each (row, group, quarter) once");
}

// ---------------------------------------------------------------- decode GEMM (17-64 rows)
void replay_dgemm(int M, int N, int K, int cus, int pk, bool swiglu, const Mut& mu) {
  const Plan p = make_plan_for(M, N, K, cus);
  if (!p.dgemm) return;
  if (swiglu && N % 2 != 0) return;
  const int G = K / BK, T = kDgT, W = kDgW, COLS = kDgCols, HT = T / 2, F = N / 2;
  const int gx = swiglu ? (F + COLS / 2 - 1) / (COLS / 2) : (N + COLS - 1) / COLS;
  const int D = dg_depth(p.rt);
  const size_t nscale = static_cast<size_t>(N) * G;
  Cover cov(N, G);
  std::vector<unsigned char> fcov(swiglu ? F : 0, 0);
  for (int by = 0; by < p.splits; ++by) {
    const int gsplit = by * p.groups_per_split;
    const int gcount = ix::imin(G, gsplit + p.groups_per_split) - gsplit;
    CHECK(gcount >= 1 && gcount <= kDgScaleGroups, "split within the scale stage", gcount,
          kDgScaleGroups);
    const int nloop = (gcount + D - 1) / D * D;
    for (int bx = 0; bx < gx; ++bx) {
      for (int c = 0; c < COLS; ++c)
        for (int gi = 0; gi < gcount; ++gi) {
          const size_t at =
              static_cast<size_t>(ix::dgemm_row(c, bx, T, W, N, swiglu)) * G + gsplit + gi;
          CHECK(at < nscale, "scale stage read", at, nscale);
        }
      for (int wave = 0; wave < W; ++wave)
        for (int lane = 0; lane < 64; ++lane) {
          const int lcol = lane & 15, q = lane >> 4;
          int rows[kDgT];
          for (int j = 0; j < T; ++j) {
            const int c = (wave * T + j) * 16 + lcol;
            const int row = ix::dgemm_row(c, bx, T, W, N, swiglu);
            rows[j] = row;
            const size_t base = woff(mu, pk, row, K, lane);
            // group i of the split, clamped to its last group for the ring's tail loads
            for (int i = 0; i < nloop + D - 1; ++i) {
              const int g = gsplit + ix::imin(i, gcount - 1);
              check_wload(pk, base + static_cast<size_t>(g) * ix::wgroup_step(pk), N, K, row,
                          64L * g + 16 * q);
              bool live_col;
              if (!swiglu) {
                live_col = bx * COLS + c < N;
              } else {
                const int f = bx * (COLS / 2) + (wave * HT + j % HT) * 16 + lcol;
                live_col = f < F;
              }
              if (i < gcount && live_col) cov.hit(row, g, q);
            }
          }
          if (swiglu)
            for (int j = 0; j < HT; ++j) {
              const int f = bx * (COLS / 2) + (wave * HT + j) * 16 + lcol;
              if (f >= F) continue;
              CHECK(rows[j] == f && rows[j + HT] == f + F, "SwiGLU gate/up pair of a lane",
                    rows[j], f);
              if (by == 0 && lane < 16) ++fcov[f];
            }
        }
    }
  }
  cov.expect_once("decode GEMM reads each (row, group, quarter) once");
  for (int f = 0; f < static_cast<int>(fcov.size()); ++f)
    if (fcov[f] != 1) {
      CHECK(false, "SwiGLU feature produced once", f, fcov[f]);
      break;
    }
}

// ---------------------------------------------------------------- prefill GEMM (>= 33 rows)
template <int WM, int WN, int TM, int TN, int STAGES, int GPS>
void replay_gemm_t(int M, int N, int K, const Plan& p, int pk, bool swiglu, const Mut& mu) {
  using T = PTile<WM, WN, TM, TN, STAGES, GPS>;
  const int G = K / BK, nsteps = K / T::KB, F = N / 2;
  const int cols = swiglu ? (F + T::BN / 2 - 1) / (T::BN / 2) : (N + T::BN - 1) / T::BN;
  const int Y = (M + T::BM - 1) / T::BM, Z = p.splits;
  CHECK(K % T::KB == 0, "K in whole stages", K, T::KB);
  // XCD order: a bijection on the grid
  {
    std::vector<unsigned char> seen(static_cast<size_t>(cols) * Y * Z, 0);
    for (int bz = 0; bz < Z; ++bz)
      for (int by = 0; by < Y; ++by)
        for (int bx = 0; bx < cols; ++bx) {
          const ix::Tile3 t = ix::gemm_tile(bx, by, bz, cols, Y, Z, SQ8_GEMM_GM);
          const bool in = t.x >= 0 && t.x < cols && t.y >= 0 && t.y < Y && t.z >= 0 && t.z < Z;
          CHECK(in, "tile coordinates inside the grid", t.x, t.y);
          if (in) ++seen[(static_cast<size_t>(t.z) * Y + t.y) * cols + t.x];
        }
    long bad = 0;
    for (unsigned char v : seen) bad += v != 1;
    CHECK(bad == 0, "XCD tile order is a bijection", bad, seen.size());
  }
  // LDS swizzle: over a stage, the slots of all threads load each (row, chunk) once.
  {
    std::vector<unsigned char> seen(static_cast<size_t>(T::BN) * T::CW, 0);
    for (int i = 0; i < T::WL; ++i)
      for (int wave = 0; wave < T::NW; ++wave)
        for (int lane = 0; lane < 64; ++lane) {
          const int slot = (i * T::NW + wave) * kWave + lane;
          const int r = slot / T::CW, q = (slot % T::CW) ^ ix::swz_w<GPS>(slot / T::CW);
          CHECK(r < T::BN && q >= 0 && q < T::CW, "weight slot inside the stage", r, q);
          if (r < T::BN && q >= 0 && q < T::CW) ++seen[static_cast<size_t>(r) * T::CW + q];
        }
    long bad = 0;
    for (unsigned char v : seen) bad += v != 1;
    CHECK(bad == 0, "weight stage chunks loaded once", bad, seen.size());
  }
  // x reads (32-bit offsets), per M tile
  for (int by = 0; by < Y; ++by) {
    const int m0 = by * T::BM;
    for (int r = 0; r < T::BM; ++r) {
      const uint64_t at = static_cast<uint64_t>(ix::imin(m0 + r, M - 1)) * K * 2 + T::CX * 16;
      CHECK(at < (1ull << 32), "x offset fits 32 bits", at, 0);
    }
  }
  Cover cov(N, G);
  std::vector<unsigned char> fcov(swiglu ? F : 0, 0);
  const size_t nscale = static_cast<size_t>(N) * G;
  for (int bz = 0; bz < Z; ++bz) {
    const int st_begin = bz * p.groups_per_split;
    const int st_end = ix::imin(nsteps, st_begin + p.groups_per_split);
    CHECK(st_end > st_begin, "split holds stages", st_begin, st_end);
    for (int bx = 0; bx < cols; ++bx) {
      for (int c = 0; c < T::BN; ++c) {
        const int row = ix::gemm_row(c, bx, T::BN, TN, N, swiglu);
        CHECK(row >= 0 && row < N, "tile column row", row, N);
        const uint64_t so = static_cast<uint64_t>(row) * G * 4;
        CHECK(so < (1ull << 32) && static_cast<size_t>(row) * G + G <= nscale, "scale offset",
              so, nscale);
        if (swiglu) {
          const int j = (c >> 5) % TN, f = ix::gemm_feat(c, bx, T::BN, TN);
          if (f < F) {
            CHECK(row == (j >= TN / 2 ? f + F : f), "SwiGLU gate/up row", row, f);
            if (bz == 0 && j < TN / 2) ++fcov[f];
          }
        }
      }
      for (int i = 0; i < T::WL; ++i)
        for (int wave = 0; wave < T::NW; ++wave)
          for (int lane = 0; lane < 64; ++lane) {
            const int slot = (i * T::NW + wave) * kWave + lane;
            const int r = slot / T::CW, q = (slot % T::CW) ^ ix::swz_w<GPS>(slot / T::CW);
            const int row = ix::gemm_row(r, bx, T::BN, TN, N, swiglu);
            const uint64_t wide =
                pk ? static_cast<uint64_t>(row >> 4) * K * 16 + (q >> 2) * 1024ull +
                         ((q & 3) * 16ull + (row & 15)) * 16ull
                   : static_cast<uint64_t>(row) * K + q * 16ull;
            uint32_t o = ix::gemm_woff(pk, static_cast<uint32_t>(row), K, q);
            if (mu.lane_place && pk)
              o = static_cast<uint32_t>((row >> 4) * K * 16 + (q >> 2) * 1024 +
                                        ((q & 3) * 16 + (r & 15)) * 16);
            CHECK(mu.lane_place || wide == o, "weight offset fits 32 bits", wide, o);
            bool live;
            if (!swiglu) live = bx * T::BN + r < N;
            else live = ix::gemm_feat(r, bx, T::BN, TN) < F;
            for (int st = st_begin; st < st_end; ++st) {
              const size_t at = static_cast<size_t>(st) * ix::gemm_stage_wstep(pk, GPS) + o;
              const long g = static_cast<long>(st) * GPS + (q >> 2);
              check_wload(pk, at, N, K, row, 64L * g + 16 * (q & 3));
              if (live) cov.hit(row, g, q & 3);
            }
          }
    }
  }
  cov.expect_once("prefill GEMM reads each (row, group, quarter) once");
  for (int f = 0; f < static_cast<int>(fcov.size()); ++f)
    if (fcov[f] != 1) {
      CHECK(false, "SwiGLU feature produced once", f, fcov[f]);
      break;
    }
}

void replay_gemm(int M, int N, int K, int cus, int pk, bool swiglu, const Mut& mu) {
  const Plan p = make_plan_for(M, N, K, cus);
  if (p.tile || p.dgemm || p.skinny) return;
  if (swiglu && N % 2 != 0) return;
  // the launcher's choice of tile (launch_mfma)
  if (p.cfg == 1 && p.gps == 1) replay_gemm_t<1, 4, 2, 2, 3, 1>(M, N, K, p, pk, swiglu, mu);
  else if (p.cfg == 1) replay_gemm_t<2, 4, 1, 2, 2, 2>(M, N, K, p, pk, swiglu, mu);
  else replay_gemm_t<2, 4, 2, 2, 3, 1>(M, N, K, p, pk, swiglu, mu);
}

struct Shape {
  const char* name;
  int N, K;
  bool swiglu;  // a fused [gate; up] weight (N = 2F) as the SwiGLU epilogue reads it
};

const Shape kShapes[] = {
    {"llama qkv", 6144, 4096, false},      {"llama o", 4096, 4096, false},
    {"llama gate/up", 28672, 4096, true},  {"llama down", 4096, 14336, false},
    {"llama lm head", 128256, 4096, false}, {"qwen2 qkv", 2048, 1536, false},
    {"qwen2 o", 1536, 1536, false},        {"qwen2 gate/up", 17920, 1536, true},
    {"qwen2 down", 1536, 8960, false},     {"qwen2 lm head", 151936, 1536, false},
    {"gate/up F=8200", 16400, 1024, true}, {"gate/up F=204", 408, 512, true},
    {"config 1", 4096, 4096, false},
};

void run(const char* tag, const std::string& ctx) {
  (void)tag;
  g_ctx = ctx;
}

int replay_all(bool quick) {
  const Mut none;
  const int Us[] = {SQ8_PGEMV_U, 8};
  // packed GEMV: every shape at 1 and 2 rows, both step widths
  for (const Shape& s : kShapes)
    for (int M = 1; M <= 2; ++M)
      for (int U : Us) {
        const bool big = static_cast<long>(s.N) * s.K > 200000000L;
        for (int cus : {256, 80, 304})
          for (int wpc : {1, 2, 4}) {
            if ((big || quick) && (cus != 256 || wpc != SQ8_PGEMV_WPC)) continue;
            run("pgemv", std::string(s.name) + " pgemv M=" + std::to_string(M) + " U=" +
                             std::to_string(U) + " cus=" + std::to_string(cus) + " wpc=" +
                             std::to_string(wpc));
            replay_pgemv(M, s.N, s.K, cus, wpc, U, none);
          }
      }
  // packed GEMV: narrow outputs and short rows
  for (int N = 1; N <= 64; ++N)
    for (int K : {256, 512, 1536, 4096, 14336})
      for (int M = 1; M <= 2; ++M)
        for (int U : Us) {
          run("pgemv", "pgemv N=" + std::to_string(N) + " K=" + std::to_string(K) + " M=" +
                           std::to_string(M) + " U=" + std::to_string(U));
          replay_pgemv(M, N, K, 256, SQ8_PGEMV_WPC, U, none);
        }
  // MFMA kernels, both weight layouts
  const int Ms[] = {3, 4, 5, 8, 9, 12, 16, 17, 24, 32, 33, 40, 48, 64, 65, 100, 128, 256, 2048};
  for (const Shape& s : kShapes)
    for (int M : Ms)
      for (int pk = 0; pk <= 1; ++pk) {
        const bool big = static_cast<long>(s.N) * s.K > 200000000L;
        if (quick && big && M != 2048 && M != 64) continue;
        const std::string c = std::string(s.name) + " M=" + std::to_string(M) + (pk ? " packed" : "");
        run("skinny", c + " skinny");
        replay_skinny(M, s.N, s.K, 256, pk, none);
        run("tile", c + " tile");
        replay_tile(M, s.N, s.K, 256, pk, none);
        for (int sw = 0; sw <= (s.swiglu ? 1 : 0); ++sw) {
          run("dgemm", c + " dgemm" + (sw ? " swiglu" : ""));
          replay_dgemm(M, s.N, s.K, 256, pk, sw, none);
          if (M >= 64 || !big) {
            run("gemm", c + " gemm" + (sw ? " swiglu" : ""));
            replay_gemm(M, s.N, s.K, 256, pk, sw, none);
          }
        }
      }
  // packed weights at 1-2 rows whose shape the packed GEMV does not take (K % 256 != 0):
  // the int8-limb skinny kernel with packed addressing
  for (int M = 1; M <= 2; ++M)
    for (int K : {64, 192, 1088, 4160}) {
      run("skinny", "packed skinny M=" + std::to_string(M) + " K=" + std::to_string(K));
      for (int N : {1, 17, 1000, 4096}) replay_skinny(M, N, K, 256, 1, none);
    }
  // other CU counts on the narrower shapes
  for (int cus : {80, 304})
    for (const Shape& s : kShapes) {
      if (static_cast<long>(s.N) * s.K > 100000000L) continue;
      for (int M : Ms)
        for (int sw = 0; sw <= (s.swiglu ? 1 : 0); ++sw) {
          run("cus", std::string(s.name) + " M=" + std::to_string(M) + " cus=" + std::to_string(cus));
          replay_skinny(M, s.N, s.K, cus, 1, none);
          replay_tile(M, s.N, s.K, cus, 1, none);
          replay_dgemm(M, s.N, s.K, cus, 1, sw, none);
          replay_gemm(M, s.N, s.K, cus, 1, sw, none);
        }
    }
  return 0;
}

// Each mutation must make the replay fail.
int mutations() {
  int missed = 0;
  g_quiet = true;
  {
    Mut mu;
    mu.scale_unclamped = true;
    const long before = g_fail;
    g_ctx = "mutation: unclamped scale read, llama o, U=8";
    replay_pgemv(1, 4096, 4096, 256, SQ8_PGEMV_WPC, 8, mu);
    const long caught = g_fail - before;
    std::printf("mutation unclamped scale read (U=8): %ld failing checks\n", caught);
    if (caught == 0) ++missed;
    g_fail = before;
  }
  {
    Mut mu;
    mu.lane_place = true;
    const long before = g_fail;
    g_ctx = "mutation: lane place";
    replay_dgemm(64, 16400, 1024, 256, 1, true, mu);
    const long c1 = g_fail - before;
    g_fail = before;
    replay_gemm(256, 16400, 1024, 256, 1, true, mu);
    const long c2 = g_fail - before;
    g_fail = before;
    std::printf("mutation lane place (F=8200 gate/up): dgemm %ld, gemm %ld failing checks\n", c1,
                c2);
    if (c1 == 0 || c2 == 0) ++missed;
  }
  g_quiet = false;
  return missed;
}

}  // namespace

int main(int argc, char** argv) {
  const bool quick = argc > 1 && std::strcmp(argv[1], "quick") == 0;
  replay_all(quick);
  const long real_fail = g_fail;
  const int missed = mutations();
  std::printf("%ld checks, %ld failures, %d mutations missed\n", g_checks, real_fail, missed);
  return real_fail == 0 && missed == 0 ? 0 : 1;
}
