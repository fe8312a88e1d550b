"""GPU parity of the HIP path (through the C ABI) against the CPU oracle.

Bar (stated once, used everywhere): against the oracle's float64 accumulation of the reference's
fp32 products (oracle sq8o_matmul_f64),
  elementwise  max |y - r| / max(|r|, 1e-3 * max|r|)  <= 1e-3
  normwise     max |y - r| / max|r|                   <= 1e-5
The reference's own fp32 order (sq8o_matmul_refgpu_f32) sits at about 1e-5 / 1e-7 on the same
metric (tests/test_oracle.py). The element-wise figure with a 1e-6 * max|r| floor
(oracle elem_err_strict) is printed beside them; the reference's own fp32 order reaches 2.6e-3 to
3.8e-2 on it at the Llama shapes, so it carries no 1e-3 bar.
"""
import zlib

import numpy as np
import pytest

from oracle import sq8_oracle as o

pytestmark = pytest.mark.gpu

ELEM_TOL = 1e-3
NORM_TOL = 1e-5

LLAMA3_8B = {"qkv": (6144, 4096), "o": (4096, 4096), "gate_up": (28672, 4096), "down": (4096, 14336)}


def run(sq8, dev, x, q, s, gs, offset_bytes=0):
    import torch
    xt = torch.from_numpy(x).to(dev)
    st = torch.from_numpy(s).to(dev)
    if offset_bytes:
        raw = torch.empty(q.size + offset_bytes, dtype=torch.int8, device=dev)
        wt = raw[offset_bytes:].view(q.shape)
        wt.copy_(torch.from_numpy(q))
    else:
        wt = torch.from_numpy(q).to(dev)
    y = sq8.matmul(xt, wt, st, group_size=gs)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def check(y, ref, label=""):
    elem, norm = o.rel_errors(y, ref)
    strict = o.elem_err_strict(y, ref)
    print(f"{label} elem={elem:.3e} norm={norm:.3e} elem_1e-6_floor={strict:.3e}", flush=True)
    assert np.all(np.isfinite(y)), label
    assert elem <= ELEM_TOL and norm <= NORM_TOL, (label, elem, norm)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 8, 13, 16, 32, 64, 65, 128, 300])
@pytest.mark.parametrize("N,K", [(8, 64), (37, 256), (200, 1024), (96, 4160)])
def test_small_shapes(sq8, dev, M, N, K):
    x, q, s = o.make_case(M, N, K, 64, seed=M * 7 + N)
    print(f"case M={M} N={N} K={K} path={sq8.path_name(M, N, K, 64)}", flush=True)
    check(run(sq8, dev, x, q, s, 64), o.matmul_f64(x, q, s, 64), f"M={M} N={N} K={K}")


@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("N,K,gs", [(33, 8192, 64), (50, 9280, 64), (17, 14336, 64),
                                    (9, 14336, 32), (21, 16000, 64), (300, 7168, 64),
                                    (19, 20480, 64), (1536, 8960, 64), (2048, 10240, 32)])
def test_long_rows_decode(sq8, dev, M, N, K, gs):
    """Decode rows of 7-20 K elements: one-row-per-wave configurations, with and without a
    partial last step, two token rows staged in up to 128 KiB of LDS, and rows whose staged
    activations exceed even that at M=2 (20480: the rows kernel)."""
    x, q, s = o.make_case(M, N, K, gs, seed=K + N + M)
    print(f"case M={M} N={N} K={K} gs={gs} path={sq8.path_name(M, N, K, gs)}", flush=True)
    check(run(sq8, dev, x, q, s, gs), o.matmul_f64(x, q, s, gs), f"M={M} N={N} K={K} gs={gs}")


@pytest.mark.parametrize("gs", [16, 32, 128, 256])
@pytest.mark.parametrize("M", [1, 4, 24, 96])
def test_other_group_sizes(sq8, dev, gs, M):
    N, K = 40, 1024
    x, q, s = o.make_case(M, N, K, gs, seed=gs + M)
    check(run(sq8, dev, x, q, s, gs), o.matmul_f64(x, q, s, gs), f"gs={gs} M={M}")


@pytest.mark.parametrize("M,N,K,gs", [(1, 5, 12, 4), (3, 7, 12, 7), (2, 16, 100, 64),
                                      (4, 10, 96, 40), (2, 33, 1000, 8)])
def test_generic_path_reference_indexing(sq8, dev, M, N, K, gs):
    """Group sizes that are not multiples of 16 or do not divide K use the reference's flat scale
    indexing (n*K)//gs + k//gs; the oracle implements the same formula."""
    rng = np.random.default_rng(M + N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal(N * K) * 0.02).astype(np.float32)
    q, s = o.quantize(w, gs)
    q = q.reshape(N, K)
    assert sq8.path_name(M, N, K, gs) == "generic"
    check(run(sq8, dev, x, q, s, gs), o.matmul_f64(x, q, s, gs), f"generic {M},{N},{K},{gs}")


@pytest.mark.parametrize("M", [1, 3, 40])
def test_unaligned_weight_pointer(sq8, dev, M):
    N, K = 24, 512
    x, q, s = o.make_case(M, N, K, 64, seed=M)
    check(run(sq8, dev, x, q, s, 64, offset_bytes=4), o.matmul_f64(x, q, s, 64), f"unaligned M={M}")


def _row_subset(N, count, seed):
    rng = np.random.default_rng(seed)
    rows = np.unique(np.concatenate([[0, N - 1], rng.choice(N, count, replace=False)]))
    return rows


@pytest.mark.parametrize("M", [1, 8, 16, 32, 48, 64, 2048])
@pytest.mark.parametrize("proj", list(LLAMA3_8B))
def test_llama3_8b_shapes(sq8, dev, proj, M):
    """Full BASELINE shapes on the GPU; the oracle checks a subset of output rows (rows are
    independent, tests/test_oracle.py::test_row_subset_equals_full)."""
    N, K = LLAMA3_8B[proj]
    x, q, s = o.make_case(M, N, K, 64, seed=zlib.crc32(f"{proj}{M}".encode()) % 1000)
    print(f"case {proj} M={M} path={sq8.path_name(M, N, K, 64)}", flush=True)
    y = run(sq8, dev, x, q, s, 64)
    rows = _row_subset(N, 48 if M >= 2048 else 200, seed=M)
    gpr = K // 64
    ref = o.matmul_f64(x, np.ascontiguousarray(q[rows]),
                       np.ascontiguousarray(s.reshape(N, gpr)[rows].reshape(-1)), 64)
    check(y[:, rows], ref, f"{proj} M={M}")


def test_lm_head_shape(sq8, dev):
    N, K = 128256, 4096
    x, q, s = o.make_case(1, N, K, 64, seed=77)
    y = run(sq8, dev, x, q, s, 64)
    rows = _row_subset(N, 300, seed=1)
    ref = o.matmul_f64(x, np.ascontiguousarray(q[rows]),
                       np.ascontiguousarray(s.reshape(N, -1)[rows].reshape(-1)), 64)
    check(y[:, rows], ref, "lm_head M=1")


def test_deterministic_and_batch_invariant_gemv(sq8, dev):
    """Same inputs give bitwise-equal outputs; on the GEMV path a batch of M rows equals M
    separate single-row calls bit for bit."""
    M, N, K = 4, 300, 4096
    x, q, s = o.make_case(M, N, K, 64, seed=5)
    y1 = run(sq8, dev, x, q, s, 64)
    y2 = run(sq8, dev, x, q, s, 64)
    np.testing.assert_array_equal(y1, y2)
    if sq8.path_name(M, N, K, 64) == sq8.path_name(1, N, K, 64):
        for m in range(M):
            np.testing.assert_array_equal(run(sq8, dev, x[m:m + 1].copy(), q, s, 64)[0], y1[m])


def test_fused_equals_separate(sq8, dev):
    """Row-stacked [wq; wk; wv] (fused QKV) gives exactly the concatenation of separate calls."""
    M, K = 8, 1024
    parts = [o.make_case(M, n, K, 64, seed=i) for i, n in enumerate((256, 64, 64))]
    x = parts[0][0]
    sep = [run(sq8, dev, x, q, s, 64) for _, q, s in parts]
    qf = np.concatenate([p[1] for p in parts])
    sf = np.concatenate([p[2] for p in parts])
    fused = run(sq8, dev, x, qf, sf, 64)
    if all(sq8.path_name(M, p[1].shape[0], K, 64) == sq8.path_name(M, qf.shape[0], K, 64) for p in parts):
        np.testing.assert_array_equal(fused, np.concatenate(sep, axis=1))
    check(fused, o.matmul_f64(x, qf, sf, 64), "fused qkv")


def test_special_values(sq8, dev):
    """Zero activations give exact zeros; a one-hot activation gives s*q exactly."""
    M, N, K = 2, 64, 512
    _, q, s = o.make_case(M, N, K, 64, seed=2)
    x = np.zeros((M, K), np.float32)
    assert np.all(run(sq8, dev, x, q, s, 64) == 0)
    x[1, 130] = 1.0
    y = run(sq8, dev, x, q, s, 64)
    exp = (s.reshape(N, -1)[:, 130 // 64] * q[:, 130].astype(np.float32)).astype(np.float32)
    np.testing.assert_array_equal(y[1], exp)


@pytest.mark.parametrize("M", [1, 3, 8, 40, 64, 100, 256])
def test_activation_dynamic_range(sq8, dev, M):
    """Token rows whose magnitudes span 1e-30 .. 1e30 each stay within tolerance of their own row
    (the f16 hi/lo split scales every row/group by its own power of two)."""
    N, K = 96, 1024
    x, q, s = o.make_case(M, N, K, 64, seed=100 + M)
    mags = np.array([1e-30, 1e-5, 1.0, 3e4, 1e30, 7e-3, 2.0, 1e10], np.float32)
    x = (x * mags[np.arange(M) % len(mags)][:, None]).astype(np.float32)
    y = run(sq8, dev, x, q, s, 64)
    ref = o.matmul_f64(x, q, s, 64)
    for m in range(M):
        check(y[m:m + 1], ref[m:m + 1], f"row {m} scale {mags[m % len(mags)]:.0e}")


def test_split_k_tickets_return_to_zero(sq8, dev):
    """Skinny split-K calls leave the workspace ticket array zero and are bitwise repeatable."""
    import torch
    M, N, K = 16, 4096, 4096
    x, q, s = o.make_case(M, N, K, 64, seed=3)
    ws = sq8.Workspace(dev)
    xt, qt, st = (torch.from_numpy(a).to(dev) for a in (x, q, s))
    ys = []
    for _ in range(3):
        ys.append(sq8.matmul(xt, qt, st, group_size=64, workspace=ws).cpu().numpy())
    torch.cuda.synchronize()
    assert int(ws.buf[:65536].count_nonzero()) == 0
    np.testing.assert_array_equal(ys[0], ys[1])
    np.testing.assert_array_equal(ys[0], ys[2])
    rows = _row_subset(N, 100, seed=4)
    ref = o.matmul_f64(x, np.ascontiguousarray(q[rows]),
                       np.ascontiguousarray(s.reshape(N, -1)[rows].reshape(-1)), 64)
    check(ys[0][:, rows], ref, "split-k M=16")


@pytest.mark.parametrize("M", [33, 48, 64])
@pytest.mark.parametrize("N,K,gs", [(300, 8192, 64), (256, 8256, 64), (200, 16384, 64),
                                    (96, 8192, 128), (130, 14336, 64)])
def test_gemm_64_row_tiles(sq8, dev, M, N, K, gs):
    """33-64 token rows with long rows go to the 64 x 256 GEMM tile: two groups per LDS stage
    when K is an even number of groups (8192, 16384, 14336), one group per stage otherwise (8256),
    group size 128 across the two groups of a stage, and split-K over few column tiles."""
    x, q, s = o.make_case(M, N, K, gs, seed=M * 11 + N + K)
    print(f"case M={M} N={N} K={K} gs={gs} fused={sq8.epilogue_fused(M, N, K, gs)}", flush=True)
    check(run(sq8, dev, x, q, s, gs), o.matmul_f64(x, q, s, gs), f"M={M} N={N} K={K} gs={gs}")


@pytest.mark.parametrize("M,N,K,gs", [(33, 16640, 1024, 64), (40, 16400, 2048, 128),
                                      (48, 16384, 4096, 64), (64, 17000, 512, 64),
                                      (17, 16400, 1024, 64), (24, 28672, 1024, 64),
                                      (32, 20000, 2048, 128)])
def test_decode_gemm_wide_outputs(sq8, dev, M, N, K, gs):
    """17-64 token rows on wide outputs take the decode GEMM (register weight ring, activation
    fragments shared through LDS): K split over several workgroups, ragged last column tiles,
    group size 128, and a split shorter than the ring."""
    x, q, s = o.make_case(M, N, K, gs, seed=M * 3 + N + K)
    print(f"case M={M} N={N} K={K} gs={gs} fused={sq8.epilogue_fused(M, N, K, gs)}", flush=True)
    check(run(sq8, dev, x, q, s, gs), o.matmul_f64(x, q, s, gs), f"M={M} N={N} K={K} gs={gs}")
