"""sq8_matmul_rmsnorm_rows: the residual add and RMSNorm ahead of the QKV and gate/up projections,
formed while the activation rows are converted for the MFMA tile and decode-GEMM kernels (one
launch fewer per projection) or, elsewhere, through the operators' own RMSNorm.

Reference: h = x + res in fp32 (the write-back, checked bit for bit), then
x' = h / sqrt(mean(h^2) + eps) * norm_w (rmsnorm_kernel.cu:8-160) in float64 and the float64
oracle product (oracle sq8o_matmul_f64), with the SwiGLU of oracle/decode_oracle.py for the
fused gate/up. Bars: the matmul's own (elementwise 1e-3 against max(|r|, 1e-3 max|r|),
normwise 1e-5).
"""
import numpy as np
import pytest

from oracle import decode_oracle as do
from oracle import sq8_oracle as o

ELEM_TOL = 1e-3
NORM_TOL = 1e-5
EPS = 1e-6


def test_rmsnorm_rows_rejects_bad_arguments(sq8):
    L = sq8.lib()
    FAKE = 4096
    assert L.sq8_matmul_rmsnorm_rows(FAKE, None, None, EPS, FAKE, FAKE, FAKE, 8, 64, 64, 64,
                                     sq8.SQ8_EPI_NONE, None, 0, None) == sq8.SQ8_ERR_NULL
    assert L.sq8_matmul_rmsnorm_rows(FAKE, None, FAKE, EPS, FAKE, FAKE, FAKE, 8, 64, 64, 64,
                                     sq8.SQ8_EPI_RESIDUAL, None, 0, None) == sq8.SQ8_ERR_DIMS
    assert L.sq8_matmul_rmsnorm_rows(FAKE, None, FAKE, EPS, FAKE, FAKE, FAKE, 8, 63, 64, 64,
                                     sq8.SQ8_EPI_SWIGLU, None, 0, None) == sq8.SQ8_ERR_DIMS
    assert L.sq8_rmsnorm_rows_fused(8, 64, 64, 64, sq8.SQ8_EPI_RESIDUAL) == 0


# (M, N, K, epilogue, with residual): tile kernel rows (9..64), the decode GEMM with its fused
# SwiGLU (33..64 rows, wide outputs), and unfused shapes (GEMV, prefill GEMM, SwiGLU behind the
# tile kernel), each with and without the residual.
CASES = [(9, 512, 1024, "none", True), (20, 1024, 4096, "none", False),
         (64, 6144, 4096, "none", True), (40, 768, 2048, "none", True),
         (64, 16384, 1024, "swiglu", True), (48, 16400, 1024, "swiglu", False),
         (1, 512, 1024, "none", True), (100, 512, 1024, "none", True),
         (100, 512, 1024, "swiglu", False), (16, 512, 1024, "swiglu", True),
         (24, 16400, 1024, "swiglu", True)]


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,epi,with_res", CASES)
def test_rmsnorm_rows_matches_oracle(sq8, dev, M, N, K, epi, with_res):
    import torch
    e = sq8.SQ8_EPI_SWIGLU if epi == "swiglu" else sq8.SQ8_EPI_NONE
    x, q, s = o.make_case(M, N, K, 64, seed=M * 7 + N + K)
    rng = np.random.default_rng(M + K)
    res = rng.standard_normal((M, K)).astype(np.float32) if with_res else None
    nw = (1.0 + 0.1 * rng.standard_normal(K)).astype(np.float32)
    fused = sq8.rmsnorm_rows_fused(M, N, K, 64, e)
    print(f"case M={M} N={N} K={K} epi={epi} res={with_res} fused={fused}", flush=True)
    dx = torch.from_numpy(x).to(dev)
    dres = torch.from_numpy(res).to(dev) if with_res else None
    dq, ds, dnw = (torch.from_numpy(a).to(dev) for a in (q, s, nw))
    F = N // 2 if e == sq8.SQ8_EPI_SWIGLU else N
    y = torch.empty((M, F), device=dev)
    sq8.matmul_rmsnorm_rows(dx, dres, dnw, EPS, dq, ds, y, e)
    torch.cuda.synchronize()
    h = x + res if with_res else x
    np.testing.assert_array_equal(dx.cpu().numpy(), h)  # written back (or left) bit for bit
    h64 = h.astype(np.float64)
    xn = h64 / np.sqrt(np.mean(h64 * h64, axis=1, keepdims=True) + EPS) * nw.astype(np.float64)
    full = o.matmul_f64(np.ascontiguousarray(xn.astype(np.float32)), q, s, 64)
    ref = do.swiglu(full[:, :F], full[:, F:]) if e == sq8.SQ8_EPI_SWIGLU else full
    got = y.cpu().numpy()
    elem, norm = o.rel_errors(got, ref)
    print(f"  elem={elem:.3e} norm={norm:.3e}", flush=True)
    assert np.all(np.isfinite(got))
    assert elem <= ELEM_TOL and norm <= NORM_TOL, (elem, norm)


@pytest.mark.gpu
def test_rmsnorm_rows_fused_paths(sq8):
    """The fused prologue covers the tile and decode-GEMM paths at the Llama-3-8B shapes."""
    E = sq8.SQ8_EPI_NONE
    assert sq8.rmsnorm_rows_fused(64, 6144, 4096, 64, E)                  # QKV, tile kernel
    assert sq8.rmsnorm_rows_fused(64, 28672, 4096, 64, sq8.SQ8_EPI_SWIGLU)  # gate/up, GEMM
    assert sq8.rmsnorm_rows_fused(16, 28672, 4096, 64, E)                 # gate/up, tile
    assert not sq8.rmsnorm_rows_fused(1, 6144, 4096, 64, E)               # GEMV
    assert not sq8.rmsnorm_rows_fused(256, 6144, 4096, 64, E)             # prefill GEMM
