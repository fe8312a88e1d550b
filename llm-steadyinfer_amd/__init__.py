"""Python binding of the gfx950 INT8 group-quant matmul library (``libsq8.so``).

The product is the C ABI in ``include/sq8.h``; this module is a thin ctypes layer used by tests
and the benchmark to call it with torch device tensors (torch supplies device memory and streams
only). There is no CPU fallback: if the HIP library is missing, ``lib()`` raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libsq8.so"

# Status codes (include/sq8.h, enum sq8_status).
SQ8_OK = 0
SQ8_ERR_NULL = -1
SQ8_ERR_DIMS = -2
SQ8_ERR_GROUP = -3
SQ8_ERR_WORKSPACE = -4
SQ8_ERR_LAUNCH = -5
SQ8_ERR_DEVICE = -6

EXPORTED_SYMBOLS = ("sq8_matmul", "sq8_workspace_bytes", "sq8_status_string", "sq8_path_name")

_lib = None


class Sq8Error(RuntimeError):
    def __init__(self, code: int):
        super().__init__(f"sq8 status {code}: {status_string(code)}")
        self.code = code


def lib() -> ctypes.CDLL:
    """Load libsq8.so (built by build.py). Import torch first so that the process shares torch's
    HIP runtime (same soname) instead of loading a second one."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"HIP library not built: {LIB_PATH} (run __graft_entry__.build())")
        L = ctypes.CDLL(str(LIB_PATH))
        vp, I, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
        L.sq8_matmul.argtypes = [vp, vp, vp, vp, I, I, I, I, vp, sz, vp]
        L.sq8_matmul.restype = I
        L.sq8_workspace_bytes.argtypes = [I, I, I, I]
        L.sq8_workspace_bytes.restype = sz
        L.sq8_status_string.argtypes = [I]
        L.sq8_status_string.restype = ctypes.c_char_p
        L.sq8_path_name.argtypes = [I, I, I, I]
        L.sq8_path_name.restype = ctypes.c_char_p
        _lib = L
    return _lib


def status_string(code: int) -> str:
    return lib().sq8_status_string(code).decode()


def path_name(M: int, N: int, K: int, group_size: int) -> str:
    return lib().sq8_path_name(M, N, K, group_size).decode()


def workspace_bytes(M: int, N: int, K: int, group_size: int) -> int:
    return int(lib().sq8_workspace_bytes(M, N, K, group_size))


def matmul_raw(x_ptr: int, w_ptr: int, s_ptr: int, y_ptr: int, M: int, N: int, K: int,
               group_size: int, ws_ptr: int = 0, ws_bytes: int = 0, stream: int = 0) -> int:
    """Call sq8_matmul with raw device addresses; returns the status code."""
    return int(lib().sq8_matmul(x_ptr or None, w_ptr or None, s_ptr or None, y_ptr or None, M, N,
                                K, group_size, ws_ptr or None, ws_bytes, stream or None))


class Workspace:
    """Grow-only device workspace for sq8_matmul (a torch uint8 tensor)."""

    def __init__(self, device="cuda"):
        self.device = device
        self.buf = None

    def get(self, nbytes: int):
        import torch
        if nbytes == 0:
            return 0, 0
        if self.buf is None or self.buf.numel() < nbytes:
            self.buf = torch.zeros(nbytes, dtype=torch.uint8, device=self.device)
        return self.buf.data_ptr(), self.buf.numel()


_default_ws = {}


def matmul(x, w, scales, y=None, group_size: int = 64, workspace: Workspace | None = None,
           stream=None):
    """y[M,N] = x[M,K] @ dequant(w[N,K], scales).T on the current torch stream.

    x: fp32 [M,K] or [K]; w: int8 [N,K]; scales: fp32 [N*K/group_size]; all on the GPU."""
    import torch
    squeeze = x.dim() == 1
    x2 = x.reshape(1, -1) if squeeze else x
    M, K = x2.shape
    N = w.shape[0]
    if y is None:
        y = torch.empty((M, N), dtype=torch.float32, device=x.device)
    for t in (x2, w, scales, y):
        if not t.is_contiguous():
            raise ValueError("sq8 tensors must be contiguous")
    if stream is None:
        stream = torch.cuda.current_stream(x.device)
    if workspace is None:
        workspace = _default_ws.setdefault(str(x.device), Workspace(x.device))
    ws_ptr, ws_n = workspace.get(workspace_bytes(M, N, K, group_size))
    rc = matmul_raw(x2.data_ptr(), w.data_ptr(), scales.data_ptr(), y.data_ptr(), M, N, K,
                    group_size, ws_ptr, ws_n, stream.cuda_stream)
    if rc != SQ8_OK:
        raise Sq8Error(rc)
    return y.reshape(-1) if squeeze else y
