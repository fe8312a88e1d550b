"""GPU tests of the packed weight layout (sq8_pack_weights and the _packed entry points),
collected after the row-major parity tests.

- The packed bytes equal a numpy restatement of the documented layout (16-row tiles, each 64-wide
  group of a tile one 1 KiB block in lane order, padding rows zero).
- From 3 token rows on the packed entry points run the row-major path's kernels with packed
  addressing, so where the row-major call takes the matrix-core path the two results are equal
  bit for bit; every result also meets the oracle bar of test_gpu_parity.py.
- At 1-2 rows the packed GEMV (and the int8-limb kernel for the shapes it does not take) is held
  to the oracle bar.
- The fused epilogue and RMSNorm-rows entry points on packed weights equal their row-major
  counterparts bit for bit where both fuse, and meet the oracle bar everywhere.
- Every call leaves the workspace's ticket area zero.
"""
import numpy as np
import pytest

from oracle import sq8_oracle as o

pytestmark = pytest.mark.gpu

ELEM_TOL = 1e-3
NORM_TOL = 1e-5
TICKET_BYTES = 64 * 1024


def pack_ref(q):
    """Packed layout of an int8 [N][K] weight, from its definition in include/sq8.h."""
    N, K = q.shape
    T, G = (N + 15) // 16, K // 64
    pad = np.zeros((T * 16, K), np.int8)
    pad[:N] = q
    # [T][16 rows][G][4 chunks][16 bytes] -> [T][G][4 chunks][16 rows][16 bytes]
    return pad.reshape(T, 16, G, 4, 16).transpose(0, 2, 3, 1, 4).reshape(-1)


def check(y, ref, label):
    elem, norm = o.rel_errors(y, ref)
    print(f"{label} elem={elem:.3e} norm={norm:.3e}", flush=True)
    assert np.all(np.isfinite(y)), label
    assert elem <= ELEM_TOL and norm <= NORM_TOL, (label, elem, norm)


def to_dev(dev, *arrs):
    import torch
    return [torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in arrs]


@pytest.mark.parametrize("N,K", [(16, 64), (37, 192), (100, 1024), (513, 256)])
def test_pack_layout(sq8, dev, N, K):
    import torch
    rng = np.random.default_rng(N + K)
    q = rng.integers(-127, 128, (N, K), dtype=np.int8)
    (qt,) = to_dev(dev, q)
    p = sq8.pack_weights(qt)
    torch.cuda.synchronize()
    assert p.data.numel() == sq8.lib().sq8_packed_weight_bytes(N, K) == ((N + 15) // 16) * 16 * K
    assert np.array_equal(p.data.cpu().numpy(), pack_ref(q))


def test_pack_rejects_bad_arguments(sq8, dev):
    import torch
    L = sq8.lib()
    q = torch.zeros((16, 96), dtype=torch.int8, device=dev)
    out = torch.empty(16 * 96, dtype=torch.int8, device=dev)
    assert L.sq8_pack_weights(q.data_ptr(), 16, 96, out.data_ptr(), None) == sq8.SQ8_ERR_DIMS
    assert L.sq8_pack_weights(None, 16, 64, out.data_ptr(), None) == sq8.SQ8_ERR_NULL
    assert L.sq8_pack_weights(q.data_ptr() + 4, 16, 64, out.data_ptr(), None) == sq8.SQ8_ERR_DIMS


def run_pair(sq8, dev, M, N, K, gs, seed):
    """(packed result, row-major result, oracle) for one case; checks the ticket area."""
    import torch
    x, q, s = o.make_case(M, N, K, gs, seed=seed)
    xt, qt, st = to_dev(dev, x, q, s)
    p = sq8.pack_weights(qt)
    ws = sq8.Workspace(dev)
    y_pk = sq8.matmul(xt, p, st, group_size=gs, workspace=ws)
    y_rm = sq8.matmul(xt, qt, st, group_size=gs)
    torch.cuda.synchronize()
    if ws.buf is not None:
        assert int(ws.buf[:TICKET_BYTES].count_nonzero()) == 0
    return y_pk.cpu().numpy(), y_rm.cpu().numpy(), o.matmul_f64(x, q, s, gs)


@pytest.mark.parametrize("M", [3, 4, 5, 8, 9, 16, 17, 24, 32, 33, 48, 64, 65, 128, 300])
@pytest.mark.parametrize("N,K", [(37, 256), (200, 1024), (520, 2048), (96, 8192),
                                 (16400, 256)])
def test_packed_equals_row_major(sq8, dev, M, N, K):
    path = sq8.path_name(M, N, K, 64)
    print(f"case M={M} N={N} K={K} row-major path={path}", flush=True)
    y_pk, y_rm, ref = run_pair(sq8, dev, M, N, K, 64, seed=M * 31 + N + K)
    check(y_pk, ref, f"packed M={M} N={N} K={K}")
    if path == "mfma":
        assert np.array_equal(y_pk, y_rm), f"M={M} N={N} K={K}"


@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("N,K,gs", [(16, 256, 64), (37, 256, 64), (200, 1024, 64),
                                    (4096, 4096, 64), (1000, 14336, 64), (9000, 512, 64),
                                    (33, 320, 64), (64, 1024, 128)])
def test_packed_few_rows(sq8, dev, M, N, K, gs):
    """1-2 rows: the packed GEMV (group 64, K % 256 == 0) or the int8-limb kernel (K = 320,
    group 128), against the oracle."""
    print(f"case M={M} N={N} K={K} gs={gs}", flush=True)
    y_pk, _, ref = run_pair(sq8, dev, M, N, K, gs, seed=M + N + K)
    check(y_pk, ref, f"packed M={M} N={N} K={K} gs={gs}")


def test_packed_unaligned_scales_take_other_kernel(sq8, dev):
    """Scales not 16-byte aligned: the 1-row call leaves the float4-scale GEMV for the int8-limb
    kernel and still meets the bar."""
    import torch
    M, N, K = 1, 48, 512
    x, q, s = o.make_case(M, N, K, 64, seed=5)
    xt, qt = to_dev(dev, x, q)
    raw = torch.empty(s.size + 1, dtype=torch.float32, device=dev)
    st = raw[1:]
    st.copy_(torch.from_numpy(s))
    y = sq8.matmul(xt, sq8.pack_weights(qt), st, group_size=64)
    torch.cuda.synchronize()
    check(y.cpu().numpy(), o.matmul_f64(x, q, s, 64), "unaligned scales")


@pytest.mark.parametrize("M", [1, 2, 8, 40, 64, 96, 300])
@pytest.mark.parametrize("epi", ["residual", "swiglu"])
def test_packed_epilogues(sq8, dev, M, epi):
    import torch
    # SwiGLU with F = N / 2 % 16 != 0 (the up rows sit at other places in their tiles than the
    # gate rows): F = 8200 on the decode GEMM (17-64 rows, N >= 16384), F = 204 on the GEMM.
    N, K = (2 * 8200, 256) if epi == "swiglu" and M in (40, 64) else (2 * 520, 1024)
    if epi == "swiglu" and M == 96:
        N = 2 * 204
    x, q, s = o.make_case(M, N, K, 64, seed=M + N)
    xt, qt, st = to_dev(dev, x, q, s)
    p = sq8.pack_weights(qt)
    code = sq8.SQ8_EPI_RESIDUAL if epi == "residual" else sq8.SQ8_EPI_SWIGLU
    cols = N if epi == "residual" else N // 2
    rng = np.random.default_rng(M)
    res = rng.standard_normal((M, cols)).astype(np.float32) if epi == "residual" else None
    outs = []
    for w in (p, qt):
        y = torch.empty((M, cols), dtype=torch.float32, device=dev)
        r = torch.from_numpy(res).to(dev) if res is not None else None
        sq8.matmul_epilogue(xt, w, st, y, code, residual=r, group_size=64)
        outs.append(y)
    torch.cuda.synchronize()
    prod = o.matmul_f64(x, q, s, 64)
    if epi == "residual":
        ref = res.astype(np.float64) + prod
    else:
        g, u = prod[:, :N // 2], prod[:, N // 2:]
        ref = g / (1 + np.exp(-g)) * u
    y_pk, y_rm = (t.cpu().numpy() for t in outs)
    check(y_pk, ref, f"packed {epi} M={M} N={N}")
    both_fused = bool(sq8.lib().sq8_epilogue_packed_fused(M, N, K, 64)) and \
        sq8.epilogue_fused(M, N, K, 64)
    print(f"fused packed/row-major: {both_fused}", flush=True)
    if both_fused:
        assert np.array_equal(y_pk, y_rm)


@pytest.mark.parametrize("M", [1, 2, 12, 40, 64, 100])
@pytest.mark.parametrize("epi", ["none", "swiglu"])
def test_packed_rmsnorm_rows(sq8, dev, M, epi):
    import torch
    N, K = (2 * 8200, 512) if epi == "swiglu" else (600, 1024)
    x, q, s = o.make_case(M, N, K, 64, seed=M + 3)
    rng = np.random.default_rng(M + 11)
    res = rng.standard_normal((M, K)).astype(np.float32)
    nw = (1 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    code = sq8.SQ8_EPI_NONE if epi == "none" else sq8.SQ8_EPI_SWIGLU
    cols = N if epi == "none" else N // 2
    qt, st, nwt = to_dev(dev, q, s, nw)
    p = sq8.pack_weights(qt)
    outs, xs = [], []
    for w in (p, qt):
        xt, rt = to_dev(dev, x, res)
        y = torch.empty((M, cols), dtype=torch.float32, device=dev)
        sq8.matmul_rmsnorm_rows(xt, rt, nwt, 1e-6, w, st, y, code, group_size=64)
        outs.append(y)
        xs.append(xt)
    torch.cuda.synchronize()
    h = x.astype(np.float64) + res
    xn = (h / np.sqrt((h * h).mean(axis=1, keepdims=True) + 1e-6) * nw).astype(np.float32)
    prod = o.matmul_f64(xn, q, s, 64)
    ref = prod if epi == "none" else prod[:, :N // 2] / (1 + np.exp(-prod[:, :N // 2])) * \
        prod[:, N // 2:]
    y_pk, y_rm = (t.cpu().numpy() for t in outs)
    check(y_pk, ref, f"packed rmsnorm {epi} M={M}")
    assert np.array_equal(xs[0].cpu().numpy(), xs[1].cpu().numpy())  # x + res written back
    if sq8.rmsnorm_rows_fused(M, N, K, 64, code) and M > 2:
        assert np.array_equal(y_pk, y_rm)


def test_packed_graph_replays_match_eager(sq8, dev):
    """One packed call per row count captured in a HIP graph and replayed with eager work
    between the replays: every replay equals the eager result."""
    import torch
    N, K = 1040, 1024
    outs = {}
    for M in (1, 2, 8, 40):
        x, q, s = o.make_case(M, N, K, 64, seed=M)
        xt, qt, st = to_dev(dev, x, q, s)
        p = sq8.pack_weights(qt)
        ws = sq8.Workspace(dev)
        y = sq8.matmul(xt, p, st, group_size=64, workspace=ws)
        torch.cuda.synchronize()
        eager = y.clone()
        g = torch.cuda.CUDAGraph()
        s2 = torch.cuda.Stream()
        s2.wait_stream(torch.cuda.current_stream())
        with torch.cuda.graph(g, stream=s2):
            sq8.matmul(xt, p, st, y, group_size=64, workspace=ws, stream=s2)
        torch.cuda.current_stream().wait_stream(s2)
        for _ in range(3):
            y.zero_()
            sq8.matmul(xt, qt, st, group_size=64)  # eager work between replays
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(y, eager), M
        outs[M] = eager


@pytest.mark.parametrize("max_batch,block_size,num_blocks", [(4, 4, 24), (96, 8, None)])
def test_packed_continuous_batching_matches_oracle(sq8, dev, tmp_path, max_batch, block_size,
                                                   num_blocks):
    """tests/test_batch.py's continuous-batching oracle test with the model on packed weights
    (every matmul through the _packed entry points): with preemption at 4 rows, and through the
    fused-epilogue GEMM at 96 rows."""
    import test_batch
    test_batch.test_continuous_batching_matches_oracle(sq8, dev, tmp_path, max_batch, block_size,
                                                       num_blocks, True, True)
