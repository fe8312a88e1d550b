"""ctypes binding and numpy helpers for the CPU oracle (test infrastructure only).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg may import this module.
The C functions are documented in sq8_oracle.c with the reference lines they restate.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "_ref" / "libsq8_oracle.so"
_lib = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_I = ctypes.c_int


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run oracle/build.py)")
        L = ctypes.CDLL(str(LIB_PATH))
        L.sq8o_quantize.argtypes = [_f32p, ctypes.c_int64, _I, _i8p, _f32p]
        L.sq8o_quantize.restype = None
        for name, yp in (("sq8o_matmul_f64", _f64p), ("sq8o_matmul_refgpu_f32", _f32p),
                         ("sq8o_matmul_cpu_loop", _f32p)):
            fn = getattr(L, name)
            fn.argtypes = [_f32p, _i8p, _f32p, yp, _I, _I, _I, _I]
            fn.restype = None
        L.sq8o_max_threads.restype = _I
        _lib = L
    return _lib


def quantize(w: np.ndarray, gs: int):
    """Group absmax quantiser (sq8o_quantize): returns (q int8 same shape, scales fp32 flat)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    if w.size % gs:
        raise ValueError("numel must be a multiple of the group size")
    q = np.empty(w.shape, np.int8)
    s = np.empty(w.size // gs, np.float32)
    lib().sq8o_quantize(w.reshape(-1), w.size, gs, q.reshape(-1), s)
    return q, s


def _check(x, q, s, gs):
    M, K = x.shape
    N, K2 = q.shape
    assert K == K2 and s.size == N * K // gs, (x.shape, q.shape, s.shape, gs)
    return M, N, K


def matmul_f64(x, q, s, gs):
    M, N, K = _check(x, q, s, gs)
    y = np.empty((M, N), np.float64)
    lib().sq8o_matmul_f64(x, q, s, y, M, N, K, gs)
    return y


def matmul_refgpu_f32(x, q, s, gs):
    M, N, K = _check(x, q, s, gs)
    y = np.empty((M, N), np.float32)
    lib().sq8o_matmul_refgpu_f32(x, q, s, y, M, N, K, gs)
    return y


def matmul_cpu_loop(x, q, s, gs):
    M, N, K = _check(x, q, s, gs)
    assert K % gs == 0
    y = np.empty((M, N), np.float32)
    lib().sq8o_matmul_cpu_loop(x, q, s, y, M, N, K, gs)
    return y


def max_threads() -> int:
    return int(lib().sq8o_max_threads())


def make_case(M: int, N: int, K: int, gs: int = 64, seed: int = 1234, w_std: float = 0.02):
    """Seeded inputs of the benchmark configs: x ~ N(0,1) fp32 [M,K]; W ~ N(0, w_std) [N,K]
    quantised to int8 with fp32 group scales."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K), dtype=np.float32)
    w = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(w_std)).astype(np.float32)
    q, s = quantize(w, gs)
    return x, q, s


def elem_err_strict(y, ref):
    """Element-wise relative error with a floor of 1e-6 * max|ref|: max |y - r| / max(|r|,
    1e-6 * max|r|). Outputs near zero dominate it: an fp32 sum over K carries an absolute error of
    order eps * sum |x w|, which next to a 1e-6 * max|r| floor is far above 1e-3 even for the
    reference kernel's own fp32 order (matmul_refgpu_f32), so it is reported beside rel_errors'
    figures, not held to their 1e-3 bar."""
    y = np.asarray(y, np.float64)
    r = np.asarray(ref, np.float64)
    amax = float(np.max(np.abs(r))) if r.size else 0.0
    if amax == 0.0:
        return float(np.max(np.abs(y))) if y.size else 0.0
    return float(np.max(np.abs(y - r) / np.maximum(np.abs(r), 1e-6 * amax)))


def rel_errors(y, ref):
    """(elementwise, normwise) relative error of y against ref.

    elementwise = max |y - r| / max(|r|, 1e-3 * max|r|); normwise = max|y - r| / max|r|."""
    y = np.asarray(y, np.float64)
    r = np.asarray(ref, np.float64)
    amax = float(np.max(np.abs(r))) if r.size else 0.0
    if amax == 0.0:
        d = float(np.max(np.abs(y))) if y.size else 0.0
        return d, d
    diff = np.abs(y - r)
    elem = float(np.max(diff / np.maximum(np.abs(r), 1e-3 * amax)))
    return elem, float(np.max(diff) / amax)
