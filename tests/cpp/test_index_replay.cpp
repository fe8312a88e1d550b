// CPU replay of the address arithmetic of the GEMV, MFMA and packed-GEMV kernels.
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
// The decode GEMV kernels (sweep, split-row) are replayed the same way for every instantiation the
// dispatch uses. Mutations of the index functions must be caught (the replay has teeth): the
// packed GEMV's scale read without its clamp at 8 groups per step (the over-read that faulted a
// lab build), a packed weight address that takes the row's place in its tile from the lane
// instead of the row, the GEMV without its tail clamp, and a split row shorter than K.
// Exit status 0 when every check passes.
#include <atomic>
#include <cstdio>
#include <functional>
#include <thread>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "sq8_plan.h"

// The split-row GEMV's chunks per wave (SQ8_GEMV_SPLITROW_U in sq8_gemv.hip, and the prologue
// variant's fixed 5).
constexpr int SQ8_GEMV_SPLITROW_U_DEFAULT = 5;

using namespace sq8;

namespace {

// Per-thread counters (tasks run on a pool of threads); each task's counts are added to the
// totals when it ends.
thread_local long g_fail = 0;
thread_local long g_checks = 0;
thread_local std::string g_ctx;
thread_local bool g_quiet = false;  // mutation runs count failures without printing them
std::atomic<long> g_printed{0};

void fail(const char* what, long long a, long long b) {
  ++g_fail;
  if (!g_quiet && g_printed.fetch_add(1) < 20)
    std::printf("FAIL [%s] %s (%lld, %lld)\n", g_ctx.c_str(), what, a, b);
}
#define CHECK(cond, what, a, b)                                  \
  do {                                                           \
    ++g_checks;                                                  \
    if (!(cond)) fail(what, (long long)(a), (long long)(b));     \
  } while (0)

// The replay as a list of independent tasks, each with the context its failures print.
struct Task {
  std::string ctx;
  std::function<void()> fn;
};
std::vector<Task> g_tasks;
void task(std::string ctx, std::function<void()> fn) {
  g_tasks.push_back(Task{std::move(ctx), std::move(fn)});
}

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

// ---------------------------------------------------------------- decode GEMV (1-4 rows)
// sweep_kernel<R, U, MT, GS, TAIL, WV, PRO, PAIR> over a grid of `grid` workgroups: each wave takes
// row blocks in grid stride and walks the row in steps of U 1 KiB chunks.
void replay_sweep(int R, int U, int WV, int MT, bool pair, int M, int N, int K, int gs, int cus,
                  int wpc, bool drop_tail = false) {
  const bool tail = !drop_tail && K % (1024 * U) != 0;
  const int nblk = ix::sw_nblk(N, R, pair);
  const int grid = ix::imin((nblk + WV - 1) / WV, (wpc / WV) * cus);
  const int GW = grid * WV, gpr = K / gs, nsteps = (K + 1024 * U - 1) / (1024 * U);
  const int X4 = MT * K / 4;  // staged float4
  CHECK(grid >= 1, "grid", grid, nblk);
  CHECK(static_cast<size_t>(MT) * K * 4 <= 128 * 1024, "activation stage", MT * K * 4, 0);
  // the stage's swizzle is a bijection on the staged float4
  {
    std::vector<unsigned char> seen(X4, 0);
    for (int i = 0; i < X4; ++i) {
      const int sl = ix::sw_xslot(i);
      CHECK(sl >= 0 && sl < X4, "stage slot", sl, X4);
      if (sl >= 0 && sl < X4) ++seen[sl];
    }
    long bad = 0;
    for (unsigned char v : seen) bad += v != 1;
    CHECK(bad == 0, "stage swizzle is a bijection", bad, X4);
  }
  std::vector<unsigned char> cov(static_cast<size_t>(N) * (K / 16), 0);
  std::vector<unsigned char> out(pair ? N / 2 : static_cast<size_t>(M) * N, 0);
  for (int gw = 0; gw < GW; ++gw) {
    int b = gw, st = 0;
    // the first step's scales are requested before the loop, then one step ahead (clamped rows)
    auto scales = [&](int bb, int ss) {
      for (int u = 0; u < U; ++u)
        for (int lane : {0, 1, 62, 63}) {  // the lanes' K offsets are affine in the lane
          const int kc = ix::sw_kc(ix::sw_k(ss * U + u, lane), K, tail);
          for (int r = 0; r < R; ++r) {
            const size_t at = static_cast<size_t>(ix::sw_row(bb, r, R, N, pair)) * gpr + kc / gs;
            CHECK(at < static_cast<size_t>(N) * gpr, "GEMV scale read", at, N * gpr);
          }
        }
    };
    scales(b, 0);
    while (b < nblk) {
      for (int u = 0; u < U; ++u)
        for (int lane = 0; lane < 64; ++lane) {
          const int k = ix::sw_k(st * U + u, lane);
          const int kc = ix::sw_kc(k, K, tail);
          CHECK(kc + 16 <= K, "GEMV weight chunk inside the row", kc, K);
          for (int r = 0; r < R; ++r) {
            const int n = ix::sw_row(b, r, R, N, pair);
            CHECK(n >= 0 && n < N, "GEMV row", n, N);
            const bool real = pair ? true : b * R + r < N;
            if (k < K && real) {
              unsigned char& v = cov[static_cast<size_t>(n) * (K / 16) + kc / 16];
              if (v < 255) ++v;
            }
          }
          for (int t = 0; t < MT; ++t) {
            const int i0 = (t * K + kc) / 4;
            for (int j = 0; j < 4; ++j) {
              const int slot = i0 + (j ^ ((i0 >> 4) & 3));  // the kernel's read
              CHECK(slot == ix::sw_xslot(i0 + j) && slot < X4, "x LDS read of float4", slot,
                    ix::sw_xslot(i0 + j));
            }
          }
        }
      int b1 = b, st1 = st + 1;
      if (st1 == nsteps) { st1 = 0; b1 += GW; }
      scales(b1, st1);
      if (st == nsteps - 1) {
        if (pair) {
          if (b < nblk) ++out[b];
        } else {
          for (int r = 0; r < R; ++r)
            for (int t = 0; t < MT; ++t)
              if (b * R + r < N && t < M) ++out[static_cast<size_t>(t) * N + b * R + r];
        }
      }
      b = b1;
      st = st1;
    }
  }
  long bad = 0;
  for (unsigned char v : cov) bad += v != 1;
  CHECK(bad == 0, "GEMV reads each 16-byte chunk of each row once", bad, cov.size());
  bad = 0;
  for (unsigned char v : out) bad += v != 1;
  CHECK(bad == 0, "GEMV writes each output once", bad, out.size());
}

// splitrow_kernel<U, KS, WV>: KS waves per row, wave part p takes chunks p, p + KS, ...
void replay_splitrow(int U, int KS, int WV, int N, int K, int gs) {
  const int RW = WV / KS;
  const int grid = (N + RW - 1) / RW;
  const bool tail = K != KS * U * 1024;
  CHECK(K <= KS * U * 1024, "split row covers K", K, KS * U * 1024);
  std::vector<unsigned char> cov(static_cast<size_t>(N) * (K / 16), 0);
  for (int bx = 0; bx < grid; ++bx)
    for (int wave = 0; wave < WV; ++wave) {
      const int rw = wave / KS, p = wave % KS;
      const int nr = ix::imin(bx * RW + rw, N - 1);
      for (int u = 0; u < U; ++u)
        for (int lane = 0; lane < 64; ++lane) {
          const int k = ix::sw_k(p + KS * u, lane);
          const int kc = ix::sw_kc(k, K, tail);
          CHECK(kc + 16 <= K && kc / gs < K / gs, "split-row chunk inside the row", kc, K);
          if (k < K && bx * RW + rw < N) {
            unsigned char& v = cov[static_cast<size_t>(nr) * (K / 16) + kc / 16];
            if (v < 255) ++v;
          }
        }
    }
  long bad = 0;
  for (unsigned char v : cov) bad += v != 1;
  CHECK(bad == 0, "split-row GEMV reads each chunk once", bad, cov.size());
}

void replay_gemv_all() {
  // every sweep_kernel instantiation the dispatch uses (launch_stream, launch_gemv,
  // launch_gemv_norm_swiglu), on every shape its preconditions allow among these
  struct Cfg { int R, U, WV, MT, wpc; bool pair; };
  const Cfg cfgs[] = {
      {1, 7, 16, 1, 16, false}, {1, 4, 8, 1, 16, false}, {1, 1, 8, 1, 16, false},
      {1, 2, 8, 1, 16, false},  {2, 1, 4, 1, 16, false}, {2, 2, 4, 1, 16, false},
      {2, 4, 4, 1, 16, false},  {1, 7, 16, 2, 16, false}, {1, 4, 8, 2, 16, false},
      {1, 1, 8, 2, 16, false},  {1, 2, 8, 2, 16, false}, {2, 1, 4, 2, 16, false},
      {2, 2, 4, 2, 16, false},  {2, 4, 4, 2, 16, false}, {1, 4, 8, 4, 16, false},
      {2, 1, 8, 1, 16, true},   {2, 2, 8, 1, 16, true},  {2, 4, 8, 1, 16, true},
  };
  const int Ns[] = {1, 3, 16, 17, 1000, 1536, 2048, 4096, 6144, 17920, 28672, 128256, 151936};
  const int Ks[] = {64, 256, 1024, 1536, 2048, 4096, 8960, 14336};
  for (const Cfg& c : cfgs)
    for (int N : Ns)
      for (int K : Ks) {
        if (static_cast<size_t>(c.MT) * K * 4 > (c.MT == 2 ? 128 * 1024 : 64 * 1024)) continue;
        if (c.pair && N % 2 != 0) continue;
        if (static_cast<long>(N) * K > 600000000L) continue;
        // wide shapes: the single-row configurations (the ones the dispatch gives them)
        if (static_cast<long>(N) * K > 50000000L && (c.MT != 1 || c.U < 4)) continue;
        for (int M = (c.MT == 4 ? 3 : c.MT); M <= c.MT; ++M) {
          task("sweep R=" + std::to_string(c.R) + " U=" + std::to_string(c.U) + " WV=" +
                   std::to_string(c.WV) + " MT=" + std::to_string(c.MT) +
                   (c.pair ? " pair" : "") + " M=" + std::to_string(M) + " N=" +
                   std::to_string(N) + " K=" + std::to_string(K),
               [=] { replay_sweep(c.R, c.U, c.WV, c.MT, c.pair, M, N, K, 64, 256, c.wpc); });
        }
      }
  for (int N : {1, 7, 1536, 2048})
    for (int K : {8192, 8960, 10240}) {
      task("splitrow N=" + std::to_string(N) + " K=" + std::to_string(K),
           [=] { replay_splitrow(SQ8_GEMV_SPLITROW_U_DEFAULT, 2, 16, N, K, 64); });
    }
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


void replay_all(bool quick) {
  const Mut none;
  replay_gemv_all();
  const int Us[] = {SQ8_PGEMV_U, 8};
  // packed GEMV: every shape at 1 and 2 rows, both step widths
  for (const Shape& s : kShapes)
    for (int M = 1; M <= 2; ++M)
      for (int U : Us) {
        const bool big = static_cast<long>(s.N) * s.K > 200000000L;
        for (int cus : {256, 80, 304})
          for (int wpc : {1, 2, 4}) {
            if ((big || quick) && (cus != 256 || wpc != SQ8_PGEMV_WPC)) continue;
            task(std::string(s.name) + " pgemv M=" + std::to_string(M) + " U=" +
                     std::to_string(U) + " cus=" + std::to_string(cus) + " wpc=" +
                     std::to_string(wpc),
                 [=] { replay_pgemv(M, s.N, s.K, cus, wpc, U, none); });
          }
      }
  // packed GEMV: narrow outputs and short rows
  for (int N = 1; N <= 64; ++N)
    for (int K : {256, 512, 1536, 4096, 14336})
      for (int M = 1; M <= 2; ++M)
        for (int U : Us) {
          task("pgemv N=" + std::to_string(N) + " K=" + std::to_string(K) + " M=" +
                   std::to_string(M) + " U=" + std::to_string(U),
               [=] { replay_pgemv(M, N, K, 256, SQ8_PGEMV_WPC, U, none); });
        }
  // MFMA kernels, both weight layouts
  const int Ms[] = {3, 4, 5, 8, 9, 12, 16, 17, 24, 32, 33, 40, 48, 64, 65, 100, 128, 256, 2048};
  for (const Shape& s : kShapes)
    for (int M : Ms)
      for (int pk = 0; pk <= 1; ++pk) {
        const bool big = static_cast<long>(s.N) * s.K > 200000000L;
        if (quick && big && M != 2048 && M != 64) continue;
        const std::string c = std::string(s.name) + " M=" + std::to_string(M) + (pk ? " packed" : "");
        task(c + " skinny", [=] { replay_skinny(M, s.N, s.K, 256, pk, none); });
        task(c + " tile", [=] { replay_tile(M, s.N, s.K, 256, pk, none); });
        for (int sw = 0; sw <= (s.swiglu ? 1 : 0); ++sw) {
          task(c + " dgemm" + (sw ? " swiglu" : ""),
               [=] { replay_dgemm(M, s.N, s.K, 256, pk, sw, none); });
          if (M >= 64 || !big)
            task(c + " gemm" + (sw ? " swiglu" : ""),
                 [=] { replay_gemm(M, s.N, s.K, 256, pk, sw, none); });
        }
      }
  // packed weights at 1-2 rows whose shape the packed GEMV does not take (K % 256 != 0):
  // the int8-limb skinny kernel with packed addressing
  for (int M = 1; M <= 2; ++M)
    for (int K : {64, 192, 1088, 4160}) {
      task("packed skinny M=" + std::to_string(M) + " K=" + std::to_string(K), [=] {
        for (int N : {1, 17, 1000, 4096}) replay_skinny(M, N, K, 256, 1, none);
      });
    }
  // other CU counts on the narrower shapes
  for (int cus : {80, 304})
    for (const Shape& s : kShapes) {
      if (static_cast<long>(s.N) * s.K > 100000000L) continue;
      for (int M : Ms)
        for (int sw = 0; sw <= (s.swiglu ? 1 : 0); ++sw) {
          task(std::string(s.name) + " M=" + std::to_string(M) + " cus=" + std::to_string(cus),
               [=] {
                 replay_skinny(M, s.N, s.K, cus, 1, none);
                 replay_tile(M, s.N, s.K, cus, 1, none);
                 replay_dgemm(M, s.N, s.K, cus, 1, sw, none);
                 replay_gemm(M, s.N, s.K, cus, 1, sw, none);
               });
        }
    }
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
  {
    const long before = g_fail;
    g_ctx = "mutation: GEMV without its tail clamp";
    replay_sweep(1, 2, 8, 1, false, 1, 1536, 1536, 64, 256, 16, /*drop_tail=*/true);
    const long c1 = g_fail - before;
    g_fail = before;
    replay_splitrow(4, 2, 16, 1536, 8960, 64);  // 8 KiB of chunks for 8.75 KiB rows
    const long c2 = g_fail - before;
    g_fail = before;
    std::printf("mutation GEMV tail (K=1536, 2 KiB steps): %ld; split row short of K: %ld "
                "failing checks\n", c1, c2);
    if (c1 == 0 || c2 == 0) ++missed;
  }
  g_quiet = false;
  return missed;
}

}  // namespace

int main(int argc, char** argv) {
  const bool quick = argc > 1 && std::strcmp(argv[1], "quick") == 0;
  replay_all(quick);
  // Largest tasks first, then a pool of threads (the hardware's count, at most 16) pulls them.
  std::atomic<size_t> next{0};
  std::atomic<long> fails{0}, checks{0};
  const unsigned hw = std::thread::hardware_concurrency();
  const unsigned nt = hw == 0 ? 4 : (hw > 16 ? 16 : hw);
  std::vector<std::thread> pool;
  for (unsigned t = 0; t < nt; ++t)
    pool.emplace_back([&] {
      for (size_t i = next.fetch_add(1); i < g_tasks.size(); i = next.fetch_add(1)) {
        g_ctx = g_tasks[i].ctx;
        g_tasks[i].fn();
      }
      fails += g_fail;
      checks += g_checks;
    });
  for (std::thread& t : pool) t.join();
  const long real_fail = fails.load();
  const int missed = mutations();
  std::printf("%zu tasks on %u threads, %ld checks, %ld failures, %d mutations missed\n",
              g_tasks.size(), nt, checks.load() + g_checks, real_fail, missed);
  return real_fail == 0 && missed == 0 ? 0 : 1;
}
