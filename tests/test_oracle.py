"""Pins of the CPU oracle (oracle/sq8_oracle.c) that need no GPU.

Each check is chosen so that a plausible slip in the oracle (wrong scale index, dropped scale,
transposed weight, wrong rounding, wrong summation order) fails at least one of them.
"""
import numpy as np
import pytest

from oracle import sq8_oracle as o


def dequant(q, s, gs):
    """Dequantised weight in float64 via the flat group index (n*K + k) // gs."""
    N, K = q.shape
    flat_idx = np.arange(N * K, dtype=np.int64) // gs
    return (q.astype(np.float64).reshape(-1) * s.astype(np.float64)[flat_idx]).reshape(N, K)


# ---------------------------------------------------------------- quantiser invariants
@pytest.mark.parametrize("gs", [16, 32, 64, 128])
def test_quantizer_invariants(gs):
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((33, 256)) * 0.02).astype(np.float32)
    q, s = o.quantize(w, gs)
    assert q.dtype == np.int8 and s.dtype == np.float32
    assert np.all(np.abs(q.astype(np.int32)) <= 127)
    groups_q = np.abs(q.reshape(-1, gs).astype(np.int32))
    groups_w = np.abs(w.reshape(-1, gs))
    # each nonzero group reaches |q| = 127 exactly at its absmax element
    assert np.all(groups_q.max(axis=1) == 127)
    np.testing.assert_array_equal(s, (groups_w.max(axis=1) / np.float32(127)).astype(np.float32))
    # reconstruction error at most half a step (plus fp32 rounding of w/s)
    err = np.abs(w.reshape(-1, gs).astype(np.float64) - q.reshape(-1, gs) * s[:, None].astype(np.float64))
    assert np.all(err <= s[:, None] * (0.5 + 1e-5))
    # signs are preserved
    assert np.all(np.sign(q.astype(np.int32)) * np.sign(w) >= 0)


def test_quantizer_round_half_away_and_zero_group():
    # group of 4: absmax 127 -> s = 1; values on .5 boundaries round away from zero
    w = np.array([127.0, 2.5, -2.5, 0.49999997, 0, 0, 0, 0], np.float32)
    q, s = o.quantize(w, 4)
    assert s[0] == np.float32(1.0) and s[1] == 0.0
    assert q.tolist() == [127, 3, -3, 0, 0, 0, 0, 0]


# ---------------------------------------------------------------- f64 golden matmul
@pytest.mark.parametrize("M,N,K,gs", [(1, 3, 64, 64), (3, 5, 128, 64), (8, 17, 192, 64),
                                      (2, 7, 96, 32), (2, 16, 100, 64), (1, 7, 12, 7)])
def test_f64_matches_numpy_dequant_matmul(M, N, K, gs):
    """numpy float64 matmul of the dequantised weight (a library routine) agrees with the oracle.
    (2,16,100,64) and (1,7,12,7) have K % gs != 0; there the reference's row offset (n*K)//gs
    equals the flat index (n*K + k)//gs only up to a carry, so compare with the reference formula."""
    rng = np.random.default_rng(M * 1000 + N)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    numel = N * K
    if numel % gs:
        pytest.skip("numel not divisible by group size")
    q, s = o.quantize(w.reshape(-1), gs)
    q = q.reshape(N, K)
    y = o.matmul_f64(x, q, s, gs)
    # reference scale index (matmul_kernel.cu:77,86)
    sidx = (np.arange(N)[:, None] * K) // gs + np.arange(K)[None, :] // gs
    xs = x[:, None, :] * s[sidx][None, :, :]  # fp32 products x*s as the reference forms them
    ref = np.einsum("mnk,nk->mn", xs.astype(np.float64), q.astype(np.float64))
    np.testing.assert_allclose(y, ref, rtol=1e-12, atol=1e-12)
    if K % gs == 0:
        ref2 = x.astype(np.float64) @ dequant(q, s, gs).T
        np.testing.assert_allclose(y, ref2, rtol=0, atol=1e-6 * np.abs(ref2).max())


def test_one_hot_known_answer():
    """x = e_k gives y[n] = s[n, k/gs] * q[n, k] exactly."""
    M, N, K, gs = 1, 9, 256, 64
    _, q, s = o.make_case(M, N, K, gs, seed=3)
    for k in (0, 63, 64, 200, 255):
        x = np.zeros((1, K), np.float32)
        x[0, k] = 1.0
        exp = s.reshape(N, K // gs)[:, k // gs].astype(np.float64) * q[:, k]
        np.testing.assert_array_equal(o.matmul_f64(x, q, s, gs)[0], exp)
        for fn in (o.matmul_refgpu_f32, o.matmul_cpu_loop):
            np.testing.assert_array_equal(fn(x, q, s, gs)[0], exp.astype(np.float32))


def test_all_ones_weight_single_scale():
    """q = 1 everywhere with one scale value: y = s * sum(x)."""
    M, N, K, gs = 2, 4, 128, 64
    x = np.arange(M * K, dtype=np.float32).reshape(M, K) / 64
    q = np.ones((N, K), np.int8)
    s = np.full(N * K // gs, 0.25, np.float32)
    y = o.matmul_f64(x, q, s, gs)
    np.testing.assert_allclose(y, 0.25 * x.astype(np.float64).sum(1)[:, None].repeat(N, 1), rtol=1e-15)


def test_zero_negation_and_scale_doubling():
    M, N, K, gs = 3, 8, 192, 64
    x, q, s = o.make_case(M, N, K, gs, seed=11)
    assert np.all(o.matmul_f64(np.zeros_like(x), q, s, gs) == 0)
    y = o.matmul_f64(x, q, s, gs)
    np.testing.assert_array_equal(o.matmul_f64(x, (-q.astype(np.int16)).astype(np.int8), s, gs), -y)
    # doubling one group's scale adds exactly that group's contribution once more
    s2 = s.copy()
    n, g = 5, 1
    s2[n * (K // gs) + g] *= 2
    y2 = o.matmul_f64(x, q, s2, gs)
    contrib = (x[:, g * gs:(g + 1) * gs].astype(np.float64) * s[n * (K // gs) + g]) @ q[n, g * gs:(g + 1) * gs]
    np.testing.assert_allclose(y2[:, n] - y[:, n], contrib, rtol=1e-6, atol=1e-9)
    other = [i for i in range(N) if i != n]
    np.testing.assert_array_equal(y2[:, other], y[:, other])


def test_weight_not_transposed():
    """A non-square case where swapping the roles of N and K cannot even run: y[m, n] uses row n."""
    M, N, K, gs = 1, 3, 128, 64
    x = np.zeros((M, K), np.float32)
    x[0, :64] = 1.0
    q = np.zeros((N, K), np.int8)
    q[2, :64] = 1
    s = np.ones(N * K // gs, np.float32)
    assert o.matmul_f64(x, q, s, gs)[0].tolist() == [0.0, 0.0, 64.0]


# ---------------------------------------------------------------- fp32 variants
def test_refgpu_order_pinned():
    """The reference reduction is a 32-lane shuffle-down tree per warp; with per-thread partials
    p0 = 1e8, p1 = 1, p2 = -1e8, p3 = 1 (others 0) the tree computes (p0 + p1) + (p2 + p3), which
    in fp32 is 1e8 + (-1e8) = 0, while a left-to-right sum would give 1."""
    K, gs = 128, 128
    x = np.zeros((1, K), np.float32)
    x[0, :4] = [1e8, 1.0, -1e8, 1.0]
    q = np.ones((1, K), np.int8)
    s = np.ones(1, np.float32)
    assert o.matmul_refgpu_f32(x, q, s, gs)[0, 0] == 0.0
    assert o.matmul_f64(x, q, s, gs)[0, 0] == 2.0
    # partials in different warps are added warp by warp: warp0 = 1e8, warp1 = 1, warp2 = -1e8
    x[:] = 0
    x[0, 0], x[0, 32], x[0, 64] = 1e8, 1.0, -1e8
    assert o.matmul_refgpu_f32(x, q, s, gs)[0, 0] == 0.0  # (1e8 + 1) - 1e8 in fp32
    x[0, 0], x[0, 32], x[0, 64] = 1e8, -1e8, 1.0
    assert o.matmul_refgpu_f32(x, q, s, gs)[0, 0] == 1.0


def test_refgpu_exact_on_integers():
    """Integer data with small sums is exact in fp32 whatever the order."""
    rng = np.random.default_rng(5)
    M, N, K, gs = 2, 6, 320, 64
    x = rng.integers(-3, 4, (M, K)).astype(np.float32)
    q = rng.integers(-127, 128, (N, K)).astype(np.int8)
    s = rng.integers(1, 4, N * K // gs).astype(np.float32)
    exact = o.matmul_f64(x, q, s, gs)
    np.testing.assert_array_equal(o.matmul_refgpu_f32(x, q, s, gs), exact.astype(np.float32))
    np.testing.assert_array_equal(o.matmul_cpu_loop(x, q, s, gs), exact.astype(np.float32))


@pytest.mark.parametrize("M,N,K", [(1, 64, 4096), (4, 32, 14336), (8, 48, 1536)])
def test_fp32_variants_within_tolerance(M, N, K):
    x, q, s = o.make_case(M, N, K, 64, seed=M + N)
    ref = o.matmul_f64(x, q, s, 64)
    for fn in (o.matmul_refgpu_f32, o.matmul_cpu_loop):
        elem, norm = o.rel_errors(fn(x, q, s, 64), ref)
        assert elem < 1e-3 and norm < 1e-5, (fn.__name__, elem, norm)


def test_row_subset_equals_full():
    """Rows are independent: slicing W rows and their scales slices y's columns (used by the GPU
    tests to check full-size shapes on a subset of rows)."""
    x, q, s = o.make_case(2, 40, 256, 64, seed=9)
    full = o.matmul_f64(x, q, s, 64)
    rows = np.array([0, 7, 39])
    sub = o.matmul_f64(x, q[rows].copy(), s.reshape(40, -1)[rows].reshape(-1).copy(), 64)
    np.testing.assert_array_equal(sub, full[:, rows])


def test_strict_elementwise_metric():
    """elem_err_strict floors |r| at 1e-6 * max|r| (the element-wise figure the parity prints
    carry beside rel_errors'): hand values, then the fact that sets its role: the reference
    kernel's own fp32 order exceeds 1e-3 on it at a Llama-3-8B shape (outputs near zero)."""
    r = np.array([[1000.0, 1e-9, -2.0]])
    y = np.array([[1000.5, 0.0, -2.0]])
    # floor 1e-3: |0.5|/1000 = 5e-4, |1e-9|/1e-3 = 1e-6, 0
    assert o.elem_err_strict(y, r) == pytest.approx(5e-4)
    y2 = np.array([[1000.0, 1e-3, -2.0]])
    assert o.elem_err_strict(y2, r) == pytest.approx((1e-3 - 1e-9) / 1e-3)
    assert o.elem_err_strict(np.zeros((1, 2)), np.zeros((1, 2))) == 0.0
    x, q, s = o.make_case(1, 4096, 4096, 64, seed=7)
    ref = o.matmul_f64(x, q, s, 64)
    refgpu = o.matmul_refgpu_f32(x, q, s, 64)
    strict = o.elem_err_strict(refgpu, ref)
    elem, norm = o.rel_errors(refgpu, ref)
    assert strict > 1e-3 > elem and norm < 1e-6
