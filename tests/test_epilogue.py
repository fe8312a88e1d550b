"""GPU parity of sq8_matmul_epilogue: the residual add and the SwiGLU of a fused [w1; w3] weight
applied in the matmul's output stage (prefill GEMM) or after it (decode paths).

References: the float64 oracle product (oracle sq8o_matmul_f64), followed by
  residual:  y = r + x.W^T                        (AddLayer after wo / w2, llama3.cpp:1139-1179)
  SwiGLU:    y = silu(x.w1^T) * (x.w3^T)           (swiglu_kernel.cu; silu(g) = g / (1 + e^-g))
computed in float64 (oracle/decode_oracle.py swiglu). Bars: the matmul's own (elementwise 1e-3
against max(|r|, 1e-3 max|r|), normwise 1e-5); structural checks are bitwise where the kernels
guarantee it (the fused residual equals matmul-then-add exactly: same accumulation, one final
add).
"""
import numpy as np
import pytest

from oracle import decode_oracle as do
from oracle import sq8_oracle as o

pytestmark = pytest.mark.gpu

ELEM_TOL = 1e-3
NORM_TOL = 1e-5


def check(y, ref, label):
    elem, norm = o.rel_errors(y, ref)
    print(f"{label} elem={elem:.3e} norm={norm:.3e}", flush=True)
    assert np.all(np.isfinite(y)), label
    assert elem <= ELEM_TOL and norm <= NORM_TOL, (label, elem, norm)


def to_dev(dev, *arrs):
    import torch
    return [torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in arrs]


# (M, F, K): the GEMM path with one split and with split-K (few tiles), features not a multiple
# of the 128-feature workgroup, the decode paths (GEMV, skinny, tile) that apply the epilogue
# after the product, and the decode GEMM (33-64 rows, wide outputs), which fuses it.
SWIGLU_CASES = [(65, 256, 1024), (128, 200, 4096), (300, 512, 256), (2048, 128, 1024),
                (1, 384, 1024), (4, 160, 2048), (8, 256, 4096), (16, 512, 1024), (33, 96, 8192),
                (48, 8200, 1024), (64, 8192, 512), (24, 8200, 1024)]


@pytest.mark.parametrize("M,F,K", SWIGLU_CASES)
def test_swiglu_epilogue(sq8, dev, M, F, K):
    import torch
    x, q, s = o.make_case(M, 2 * F, K, 64, seed=M + 3 * F + K)
    print(f"case swiglu M={M} F={F} K={K} fused={sq8.epilogue_fused(M, 2 * F, K)}", flush=True)
    xt, qt, st = to_dev(dev, x, q, s)
    y = torch.empty((M, F), dtype=torch.float32, device=dev)
    sq8.matmul_epilogue(xt, qt, st, y, sq8.SQ8_EPI_SWIGLU)
    torch.cuda.synchronize()
    full = o.matmul_f64(x, q, s, 64)
    ref = do.swiglu(full[:, :F], full[:, F:])
    check(y.cpu().numpy(), ref, f"swiglu M={M} F={F} K={K}")
    # same product through sq8_matmul, then the SwiGLU rows operator: agrees to fp32 rounding
    gu = sq8.matmul(xt, qt, st)
    h = torch.empty_like(y)
    sq8.swiglu_rows(gu, h)
    torch.cuda.synchronize()
    d = (y - h).abs().max().item() / max(h.abs().max().item(), 1e-30)
    assert d <= 1e-6, d


RESID_CASES = [(65, 512, 1024), (128, 4096, 4096), (300, 1000, 2048), (2048, 256, 1024),
               (1, 512, 1024), (8, 4096, 4096), (16, 1024, 1024), (40, 4096, 14336),
               (64, 16384, 512), (36, 16400, 1024)]


@pytest.mark.parametrize("M,N,K", RESID_CASES)
@pytest.mark.parametrize("inplace", [False, True])
def test_residual_epilogue(sq8, dev, M, N, K, inplace):
    import torch
    x, q, s = o.make_case(M, N, K, 64, seed=M * 5 + N + K)
    r = np.random.default_rng(M + N).standard_normal((M, N)).astype(np.float32)
    print(f"case residual M={M} N={N} K={K} inplace={inplace} "
          f"fused={sq8.epilogue_fused(M, N, K)}", flush=True)
    xt, qt, st, rt = to_dev(dev, x, q, s, r)
    y = rt.clone() if inplace else torch.empty((M, N), dtype=torch.float32, device=dev)
    sq8.matmul_epilogue(xt, qt, st, y, sq8.SQ8_EPI_RESIDUAL, residual=y if inplace else rt)
    torch.cuda.synchronize()
    ref = r.astype(np.float64) + o.matmul_f64(x, q, s, 64)
    check(y.cpu().numpy(), ref, f"residual M={M} N={N} K={K}")
    plain = sq8.matmul(xt, qt, st)
    torch.cuda.synchronize()
    assert torch.equal(y, rt + plain)


def test_llama_shapes_row_subset(sq8, dev):
    """Prefill chunk at the Llama-3-8B gate/up and down shapes: the fused epilogues against the
    oracle on a subset of output columns (columns are independent)."""
    import torch
    M, K, F = 256, 4096, 14336
    x, q, s = o.make_case(M, 2 * F, K, 64, seed=77)
    xt, qt, st = to_dev(dev, x, q, s)
    y = torch.empty((M, F), dtype=torch.float32, device=dev)
    sq8.matmul_epilogue(xt, qt, st, y, sq8.SQ8_EPI_SWIGLU)
    torch.cuda.synchronize()
    cols = np.arange(0, F, 97)
    rows = np.concatenate([cols, cols + F])
    gs_per_row = K // 64
    srows = s.reshape(2 * F, gs_per_row)[rows].reshape(-1)
    full = o.matmul_f64(x, q[rows], srows, 64)
    ref = do.swiglu(full[:, :len(cols)], full[:, len(cols):])
    check(y.cpu().numpy()[:, cols], ref, "swiglu llama gate/up M=256")
