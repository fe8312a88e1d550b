"""Python binding of the gfx950 INT8 group-quant matmul library (``libsq8.so``).

The product is the C ABI in ``include/sq8.h``; this module is a thin ctypes layer used by tests
and the benchmark to call it with torch device tensors (torch supplies device memory and streams
only). There is no CPU fallback: if the HIP library is missing, ``lib()`` raises.
"""
from __future__ import annotations

import ctypes
import math
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

EXPORTED_SYMBOLS = ("sq8_matmul", "sq8_workspace_bytes", "sq8_status_string", "sq8_path_name",
                    "sq8_matmul_epilogue", "sq8_epilogue_workspace_bytes", "sq8_epilogue_fused",
                    "sq8_matmul_rmsnorm_rows", "sq8_rmsnorm_rows_fused",
                    "sq8_rmsnorm_rows_workspace_bytes", "sq8_matmul_noalloc",
                    "sq8_noalloc_scratch_bytes", "sq8_packed_weight_bytes", "sq8_pack_weights",
                    "sq8_packed_workspace_bytes", "sq8_matmul_packed",
                    "sq8_epilogue_packed_fused", "sq8_epilogue_packed_workspace_bytes",
                    "sq8_matmul_epilogue_packed", "sq8_rmsnorm_rows_packed_workspace_bytes",
                    "sq8_matmul_rmsnorm_rows_packed")

# Output epilogues (include/sq8.h, enum sq8_epilogue).
SQ8_EPI_NONE = 0
SQ8_EPI_RESIDUAL = 1
SQ8_EPI_SWIGLU = 2
# include/sq8_decode.h
DECODE_SYMBOLS = ("sq8_embedding", "sq8_rmsnorm", "sq8_add_rmsnorm", "sq8_rope_tables", "sq8_rope_kv",
                  "sq8_attention_decode", "sq8_swiglu", "sq8_add", "sq8_argmax_workspace_bytes",
                  "sq8_argmax", "sq8_quantize", "sq8_step_advance", "sq8_matmul_rmsnorm",
                  "sq8_matmul_swiglu", "sq8_rope_attention_decode", "sq8_matmul_rmsnorm_swiglu",
                  "sq8_argmax_advance", "sq8_decode_attention_workspace_bytes",
                  "sq8_rope_attention_decode_ws")
# include/sq8_batch.h
BATCH_SYMBOLS = ("sq8_paged_rope_kv", "sq8_paged_attention", "sq8_paged_attention_ws",
                 "sq8_paged_attention_workspace_bytes", "sq8_swiglu_rows", "sq8_argmax_rows")

# include/sq8_probe.h (measurement only)
PROBE_SYMBOLS = ("sq8_probe_stream_read",)

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
        L.sq8_matmul_epilogue.argtypes = [vp, vp, vp, vp, I, I, I, I, I, vp, vp, sz, vp]
        L.sq8_matmul_epilogue.restype = I
        L.sq8_epilogue_workspace_bytes.argtypes = [I, I, I, I, I]
        L.sq8_epilogue_workspace_bytes.restype = sz
        L.sq8_matmul_rmsnorm_rows.argtypes = [vp, vp, vp, ctypes.c_float, vp, vp, vp, I, I, I,
                                               I, I, vp, sz, vp]
        L.sq8_matmul_rmsnorm_rows.restype = I
        L.sq8_rmsnorm_rows_fused.argtypes = [I, I, I, I, I]
        L.sq8_rmsnorm_rows_fused.restype = I
        L.sq8_rmsnorm_rows_workspace_bytes.argtypes = [I, I, I, I, I]
        L.sq8_rmsnorm_rows_workspace_bytes.restype = sz
        L.sq8_packed_weight_bytes.argtypes = [I, I]
        L.sq8_packed_weight_bytes.restype = sz
        L.sq8_pack_weights.argtypes = [vp, I, I, vp, vp]
        L.sq8_packed_workspace_bytes.argtypes = [I, I, I, I]
        L.sq8_packed_workspace_bytes.restype = sz
        L.sq8_matmul_packed.argtypes = [vp, vp, vp, vp, I, I, I, I, vp, sz, vp]
        L.sq8_epilogue_packed_fused.argtypes = [I, I, I, I]
        L.sq8_epilogue_packed_workspace_bytes.argtypes = [I, I, I, I, I]
        L.sq8_epilogue_packed_workspace_bytes.restype = sz
        L.sq8_matmul_epilogue_packed.argtypes = [vp, vp, vp, vp, I, I, I, I, I, vp, vp, sz, vp]
        L.sq8_rmsnorm_rows_packed_workspace_bytes.argtypes = [I, I, I, I, I]
        L.sq8_rmsnorm_rows_packed_workspace_bytes.restype = sz
        L.sq8_matmul_rmsnorm_rows_packed.argtypes = [vp, vp, vp, ctypes.c_float, vp, vp, vp, I,
                                                     I, I, I, I, vp, sz, vp]
        L.sq8_epilogue_fused.argtypes = [I, I, I, I]
        L.sq8_epilogue_fused.restype = I
        f32 = ctypes.c_float
        sigs = {
            "sq8_embedding": [vp, I, I, vp, I, vp, vp],
            "sq8_rmsnorm": [vp, vp, vp, I, I, f32, vp],
            "sq8_add_rmsnorm": [vp, vp, vp, vp, I, I, f32, vp],
            "sq8_rope_tables": [vp, vp, I, I, f32, vp],
            "sq8_rope_kv": [vp, I, I, I, vp, vp, vp, vp, vp, I, vp],
            "sq8_attention_decode": [vp, vp, vp, vp, vp, I, I, I, I, vp],
            "sq8_swiglu": [vp, vp, vp, I, vp],
            "sq8_add": [vp, vp, I, vp],
            "sq8_argmax": [vp, I, vp, vp, sz, vp],
            "sq8_quantize": [vp, ctypes.c_int64, I, vp, vp, vp],
            "sq8_step_advance": [vp, vp, vp, vp],
            "sq8_matmul_rmsnorm": [vp, vp, vp, vp, f32, vp, vp, vp, I, I, I, vp],
            "sq8_matmul_swiglu": [vp, vp, vp, vp, I, I, I, vp],
            "sq8_matmul_rmsnorm_swiglu": [vp, vp, vp, vp, f32, vp, vp, vp, I, I, I, vp],
            "sq8_argmax_advance": [vp, I, vp, sz, vp, vp, vp, I, I, vp, vp],
            "sq8_rope_attention_decode_ws": [vp, I, I, I, vp, vp, vp, vp, vp, vp, I, vp, sz, vp],
            "sq8_rope_attention_decode": [vp, I, I, I, vp, vp, vp, vp, vp, vp, I, vp],
            "sq8_paged_rope_kv": [vp, I, I, I, I, vp, vp, I, I, vp, vp, vp, vp, vp],
            "sq8_paged_attention": [vp, I, I, I, I, I, vp, vp, I, I, vp, vp, vp, vp],
            "sq8_paged_attention_ws": [vp, I, I, I, I, I, vp, vp, I, I, vp, vp, vp, vp, sz, vp],
            "sq8_swiglu_rows": [vp, I, I, vp, vp],
            "sq8_argmax_rows": [vp, I, I, vp, vp],
            "sq8_matmul_noalloc": [vp, vp, vp, vp, I, I, I, I, vp],
            "sq8_probe_stream_read": [vp, sz, vp, I, I, I, vp],
        }
        for name, args in sigs.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = I
        L.sq8_decode_attention_workspace_bytes.argtypes = [I, I, I]
        L.sq8_decode_attention_workspace_bytes.restype = sz
        L.sq8_noalloc_scratch_bytes.argtypes = []
        L.sq8_noalloc_scratch_bytes.restype = sz
        L.sq8_argmax_workspace_bytes.argtypes = [I]
        L.sq8_argmax_workspace_bytes.restype = sz
        L.sq8_paged_attention_workspace_bytes.argtypes = [I, I, I, I, I, I]
        L.sq8_paged_attention_workspace_bytes.restype = sz
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


class PackedWeight:
    """An INT8 weight [N][K] in the packed layout of sq8_pack_weights (16-row tiles, each 64-wide
    group of a tile one contiguous 1 KiB block). Accepted wherever a row-major int8 weight is:
    matmul, matmul_epilogue and matmul_rmsnorm_rows then call the _packed entry points."""

    def __init__(self, data, N: int, K: int):
        self.data, self.N, self.K = data, N, K
        self.shape = (N, K)
        self.device = data.device

    def data_ptr(self) -> int:
        return self.data.data_ptr()

    def is_contiguous(self) -> bool:
        return True


def pack_weights(w, stream=None) -> PackedWeight:
    """Repack a row-major int8 weight [N][K] (K % 64 == 0) on the GPU (sq8_pack_weights)."""
    import torch
    N, K = w.shape
    if not w.is_contiguous():
        raise ValueError("sq8 tensors must be contiguous")
    data = torch.empty(int(lib().sq8_packed_weight_bytes(N, K)), dtype=torch.int8,
                       device=w.device)
    if stream is None:
        stream = torch.cuda.current_stream(w.device)
    rc = int(lib().sq8_pack_weights(w.data_ptr(), N, K, data.data_ptr(), stream.cuda_stream))
    if rc != SQ8_OK:
        raise Sq8Error(rc)
    return PackedWeight(data, N, K)


def _check_matmul(x, w, scales, y, group_size: int, out_cols: int, extra=()):
    """The shape, dtype and placement checks of MatmulLayer::check (src/source/op/matmul.cpp:
    19-77), made before anything is launched: the C ABI takes plain pointers and cannot see a
    buffer's size, so a mismatch here would become an out-of-bounds access on the GPU.
    x fp32 [M][K]; w int8 [N][K] (row-major or PackedWeight); scales fp32 [N*K/group_size];
    y fp32 [M][out_cols]; extra: (name, tensor, shape) triples (fp32) checked the same way."""
    import torch
    M, K = x.shape
    N = w.shape[0]
    if tuple(w.shape) != (N, K):
        raise ValueError(f"weight shape {tuple(w.shape)} does not match input width {K}")
    if group_size <= 0 or (N * K) % group_size != 0:
        raise ValueError(f"group size {group_size} does not divide the {N}x{K} weight")
    wdt = w.data.dtype if isinstance(w, PackedWeight) else w.dtype
    if wdt != torch.int8:
        raise ValueError(f"weight dtype {wdt}, expected torch.int8")
    f32 = torch.float32
    for name, t, n in (("input", x, M * K), ("scales", scales, N * K // group_size),
                       ("output", y, M * out_cols)) + tuple(
                           (nm, t, math.prod(sh)) for nm, t, sh in extra):
        if t.dtype != f32:
            raise ValueError(f"{name} dtype {t.dtype}, expected {f32}")
        if t.numel() != n:
            raise ValueError(f"{name} holds {t.numel()} values, expected {n}")
        if not t.is_contiguous():
            raise ValueError("sq8 tensors must be contiguous")
        if t.device != x.device:
            raise ValueError(f"{name} on {t.device}, input on {x.device}")
    if w.device != x.device:
        raise ValueError(f"weight on {w.device}, input on {x.device}")
    if x.device.type != "cuda":
        raise ValueError(f"operands on {x.device}, expected a GPU")

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
    _check_matmul(x2, w, scales, y, group_size, N)
    if stream is None:
        stream = torch.cuda.current_stream(x.device)
    if workspace is None:
        workspace = _default_ws.setdefault(str(x.device), Workspace(x.device))
    if isinstance(w, PackedWeight):
        ws_ptr, ws_n = workspace.get(int(lib().sq8_packed_workspace_bytes(M, N, K, group_size)))
        rc = int(lib().sq8_matmul_packed(x2.data_ptr(), w.data_ptr(), scales.data_ptr(),
                                         y.data_ptr(), M, N, K, group_size, ws_ptr or None, ws_n,
                                         stream.cuda_stream))
    else:
        ws_ptr, ws_n = workspace.get(workspace_bytes(M, N, K, group_size))
        rc = matmul_raw(x2.data_ptr(), w.data_ptr(), scales.data_ptr(), y.data_ptr(), M, N, K,
                        group_size, ws_ptr, ws_n, stream.cuda_stream)
    if rc != SQ8_OK:
        raise Sq8Error(rc)
    return y.reshape(-1) if squeeze else y


def epilogue_fused(M: int, N: int, K: int, group_size: int = 64, packed: bool = False) -> bool:
    if packed:
        return bool(lib().sq8_epilogue_packed_fused(M, N, K, group_size))
    return bool(lib().sq8_epilogue_fused(M, N, K, group_size))


def matmul_epilogue(x, w, scales, y, epilogue: int, residual=None, group_size: int = 64,
                    workspace: Workspace | None = None, stream=None):
    """y = epilogue(x[M,K] @ dequant(w[N,K], scales).T) through sq8_matmul_epilogue.

    SQ8_EPI_RESIDUAL: y[M,N] = residual + product (residual may be y itself).
    SQ8_EPI_SWIGLU: w is the fused [w1; w3] (N = 2F); y[M,F] = silu(gate) * up."""
    import torch
    M, K = x.shape
    N = w.shape[0]
    out_cols = N // 2 if epilogue == SQ8_EPI_SWIGLU else N
    extra = () if residual is None else (("residual", residual, (M, out_cols)),)
    _check_matmul(x, w, scales, y, group_size, out_cols, extra)
    if stream is None:
        stream = torch.cuda.current_stream(x.device)
    if workspace is None:
        workspace = _default_ws.setdefault(str(x.device), Workspace(x.device))
    pk = isinstance(w, PackedWeight)
    need = (lib().sq8_epilogue_packed_workspace_bytes if pk
            else lib().sq8_epilogue_workspace_bytes)(M, N, K, group_size, epilogue)
    ws_ptr, ws_n = workspace.get(int(need))
    fn = lib().sq8_matmul_epilogue_packed if pk else lib().sq8_matmul_epilogue
    rc = int(fn(x.data_ptr(), w.data_ptr(), scales.data_ptr(), y.data_ptr(), M, N, K, group_size,
                epilogue, _ptr(residual), ws_ptr or None, ws_n, stream.cuda_stream))
    if rc != SQ8_OK:
        raise Sq8Error(rc)
    return y


def rmsnorm_rows_fused(M: int, N: int, K: int, group_size: int = 64,
                       epilogue: int = SQ8_EPI_NONE) -> bool:
    """Whether sq8_matmul_rmsnorm_rows forms the norm inside the matmul's launches here."""
    return bool(lib().sq8_rmsnorm_rows_fused(M, N, K, group_size, epilogue))


def matmul_rmsnorm_rows(x, res, norm_w, eps: float, w, scales, y, epilogue: int = SQ8_EPI_NONE,
                        group_size: int = 64, workspace: Workspace | None = None, stream=None):
    """y = epilogue(rmsnorm(x + res) * norm_w @ dequant(w, scales).T); x + res is written back
    to x (res may be None: x is only read)."""
    import torch
    M, K = x.shape
    N = w.shape[0]
    extra = (("norm weight", norm_w, (K,)),) + (() if res is None else (("residual", res, (M, K)),))
    _check_matmul(x, w, scales, y, group_size, N // 2 if epilogue == SQ8_EPI_SWIGLU else N, extra)
    if stream is None:
        stream = torch.cuda.current_stream(x.device)
    if workspace is None:
        workspace = _default_ws.setdefault(str(x.device), Workspace(x.device))
    pk = isinstance(w, PackedWeight)
    need = (lib().sq8_rmsnorm_rows_packed_workspace_bytes if pk
            else lib().sq8_rmsnorm_rows_workspace_bytes)(M, N, K, group_size, epilogue)
    ws_ptr, ws_n = workspace.get(int(need))
    fn = lib().sq8_matmul_rmsnorm_rows_packed if pk else lib().sq8_matmul_rmsnorm_rows
    rc = int(fn(x.data_ptr(), _ptr(res), norm_w.data_ptr(), eps, w.data_ptr(), scales.data_ptr(),
                y.data_ptr(), M, N, K, group_size, epilogue, ws_ptr or None, ws_n,
                stream.cuda_stream))
    if rc != SQ8_OK:
        raise Sq8Error(rc)
    return y


# ----------------------------------------------------------------------------- decode operators
# Thin wrappers over include/sq8_decode.h taking torch device tensors; each raises Sq8Error on a
# non-zero status. `stream` defaults to torch's current stream.


def _ptr(t):
    return None if t is None else t.data_ptr()


def _call(name: str, *args, stream=None):
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    rc = int(getattr(lib(), name)(*args, stream.cuda_stream))
    if rc != SQ8_OK:
        raise Sq8Error(rc)


def embedding(table, tokens, out, stream=None):
    """out[i] = table[tokens[i]] (tokens int32 on the device)."""
    vocab, dim = table.shape
    _call("sq8_embedding", _ptr(table), vocab, dim, _ptr(tokens), tokens.numel(), _ptr(out),
          stream=stream)


def rmsnorm(x, w, out, eps: float = 1e-6, stream=None):
    dim = w.numel()
    _call("sq8_rmsnorm", _ptr(x), _ptr(w), _ptr(out), x.numel() // dim, dim, eps, stream=stream)


def add_rmsnorm(x, res, w, out, eps: float = 1e-6, stream=None):
    """x += res (in place), out = rmsnorm(x) * w."""
    dim = w.numel()
    _call("sq8_add_rmsnorm", _ptr(x), _ptr(res), _ptr(w), _ptr(out), x.numel() // dim, dim, eps,
          stream=stream)


def rope_tables(sin_cache, cos_cache, head_size: int, max_seq: int, theta: float, stream=None):
    _call("sq8_rope_tables", _ptr(sin_cache), _ptr(cos_cache), head_size, max_seq, theta,
          stream=stream)


def rope_kv(qkv, dim: int, kv_dim: int, head_size: int, pos, sin_cache, cos_cache, kcache, vcache,
            max_seq: int, stream=None):
    _call("sq8_rope_kv", _ptr(qkv), dim, kv_dim, head_size, _ptr(pos), _ptr(sin_cache),
          _ptr(cos_cache), _ptr(kcache), _ptr(vcache), max_seq, stream=stream)


def attention_decode(q, kcache, vcache, pos, out, head_num: int, kv_head_num: int, head_size: int,
                     max_seq: int, stream=None):
    _call("sq8_attention_decode", _ptr(q), _ptr(kcache), _ptr(vcache), _ptr(pos), _ptr(out),
          head_num, kv_head_num, head_size, max_seq, stream=stream)


def swiglu(a, b, out, stream=None):
    _call("sq8_swiglu", _ptr(a), _ptr(b), _ptr(out), a.numel(), stream=stream)


def add(x, y, stream=None):
    _call("sq8_add", _ptr(x), _ptr(y), x.numel(), stream=stream)


def argmax(logits, out, workspace: Workspace | None = None, stream=None):
    """out[0] = first argmax of logits (int32 on the device)."""
    n = logits.numel()
    if workspace is None:
        workspace = _default_ws.setdefault(str(logits.device) + ":argmax", Workspace(logits.device))
    ws_ptr, ws_n = workspace.get(int(lib().sq8_argmax_workspace_bytes(n)))
    _call("sq8_argmax", _ptr(logits), n, _ptr(out), ws_ptr or None, ws_n, stream=stream)


def quantize(w, q, scales, group_size: int = 64, stream=None):
    _call("sq8_quantize", _ptr(w), w.numel(), group_size, _ptr(q), _ptr(scales), stream=stream)


def step_advance(pos, token, next_token, stream=None):
    _call("sq8_step_advance", _ptr(pos), _ptr(token), _ptr(next_token), stream=stream)


def matmul_rmsnorm(x, res, x_out, norm_w, w, scales, y, group_size: int = 64, eps: float = 1e-6,
                   stream=None):
    """y = matmul(rmsnorm(x + res) * norm_w, w); x + res also written to x_out (res, x_out may be
    None)."""
    N, K = w.shape
    _call("sq8_matmul_rmsnorm", _ptr(x), _ptr(res), _ptr(x_out), _ptr(norm_w), eps, _ptr(w),
          _ptr(scales), _ptr(y), N, K, group_size, stream=stream)


def probe_stream_read(buf, sink, workgroups_per_cu: int = 8, chunks_per_lane: int = 4,
                      stream=None):
    """Read-only streaming probe over buf (any dtype, 16-byte multiple); adds the wrapping uint32
    sums of its 32-bit words into the counters of sink (an int32 device tensor)."""
    _call("sq8_probe_stream_read", _ptr(buf), buf.numel() * buf.element_size(), _ptr(sink),
          sink.numel(), workgroups_per_cu, chunks_per_lane, stream=stream)


def matmul_rmsnorm_swiglu(x, res, x_out, norm_w, w, scales, y, group_size: int = 64,
                          eps: float = 1e-6, stream=None):
    """y = silu(g) * u with [g; u] = matmul(rmsnorm(x + res) * norm_w, w) (w = [w1; w3], y of
    N/2 values); x + res also written to x_out (res, x_out may be None)."""
    N, K = w.shape
    _call("sq8_matmul_rmsnorm_swiglu", _ptr(x), _ptr(res), _ptr(x_out), _ptr(norm_w), eps,
          _ptr(w), _ptr(scales), _ptr(y), N, K, group_size, stream=stream)


def argmax_advance(logits, pos, token, emb_table, x, workspace: Workspace, stream=None):
    """*token = first argmax of logits, *pos += 1, x = emb_table[*token] (one launch)."""
    n = logits.numel()
    vocab, dim = emb_table.shape
    ws_ptr, ws_n = workspace.get(int(lib().sq8_argmax_workspace_bytes(n)))
    _call("sq8_argmax_advance", _ptr(logits), n, ws_ptr, ws_n, _ptr(pos), _ptr(token),
          _ptr(emb_table), vocab, dim, _ptr(x), stream=stream)


def matmul_swiglu(gate_up, w, scales, y, group_size: int = 64, stream=None):
    """y = matmul(silu(gate_up[:K]) * gate_up[K:], w)."""
    N, K = w.shape
    _call("sq8_matmul_swiglu", _ptr(gate_up), _ptr(w), _ptr(scales), _ptr(y), N, K, group_size,
          stream=stream)


def rope_attention_decode(qkv, head_num: int, kv_head_num: int, head_size: int, pos, sin_cache,
                          cos_cache, kcache, vcache, out, max_seq: int, workspace=None,
                          stream=None):
    """RoPE on the token's q and k, cache write at *pos and attention, in one launch. With a
    workspace (zero-filled before its first use, decode_attention_workspace_bytes() bytes) the
    positions are split over several workgroups per head."""
    if workspace is None:
        _call("sq8_rope_attention_decode", _ptr(qkv), head_num, kv_head_num, head_size,
              _ptr(pos), _ptr(sin_cache), _ptr(cos_cache), _ptr(kcache), _ptr(vcache), _ptr(out),
              max_seq, stream=stream)
    else:
        _call("sq8_rope_attention_decode_ws", _ptr(qkv), head_num, kv_head_num, head_size,
              _ptr(pos), _ptr(sin_cache), _ptr(cos_cache), _ptr(kcache), _ptr(vcache), _ptr(out),
              max_seq, _ptr(workspace), workspace.numel() * workspace.element_size(),
              stream=stream)


def decode_attention_workspace_bytes(head_num: int, head_size: int, max_seq: int) -> int:
    return int(lib().sq8_decode_attention_workspace_bytes(head_num, head_size, max_seq))


# Thin wrappers over include/sq8_batch.h (continuous batching, paged KV cache).


def _check_paged(qkv, q_width: int, head_num: int, kv_head_num: int, head_size: int, positions,
                 block_table, block_size: int, kcache, vcache, out=None):
    """Shape checks of the paged operators before launch (the kernels index every buffer from
    these sizes; the reference checks them in its batched forward, llama3.cpp:996-1062)."""
    import torch
    rows = positions.numel()
    dim, kv_dim = head_num * head_size, kv_head_num * head_size
    if head_num <= 0 or kv_head_num <= 0 or head_num % kv_head_num != 0:
        raise ValueError(f"{head_num} query heads over {kv_head_num} kv heads")
    if positions.dtype != torch.int32 or block_table.dtype != torch.int32:
        raise ValueError("positions and block tables must be int32")
    if block_table.dim() != 2 or block_table.shape[0] < rows:
        raise ValueError(f"block table {tuple(block_table.shape)} for {rows} rows")
    if q_width < dim + 2 * kv_dim or qkv.numel() < (rows - 1) * q_width + dim + 2 * kv_dim:
        raise ValueError(f"qkv of {qkv.numel()} values for {rows} rows of width {q_width}")
    for name, c in (("key cache", kcache), ("value cache", vcache)):
        if c.dim() != 3 or c.shape[1] != block_size or c.shape[2] != kv_dim:
            raise ValueError(f"{name} {tuple(c.shape)}, expected [blocks][{block_size}][{kv_dim}]")
    if out is not None and out.numel() < rows * dim:
        raise ValueError(f"output of {out.numel()} values for {rows} rows of {dim}")
    for t in (qkv, positions, block_table, kcache, vcache) + (() if out is None else (out,)):
        if not t.is_contiguous():
            raise ValueError("sq8 tensors must be contiguous")
        if t.dtype not in (torch.float32, torch.int32):
            raise ValueError(f"unexpected dtype {t.dtype}")


def paged_rope_kv(qkv, head_num: int, kv_head_num: int, head_size: int, positions, block_table,
                  block_size: int, sin_cache, cos_cache, kcache, vcache, stream=None):
    """Rows of qkv ([rows][dim + 2 kv_dim]) at their positions: rotate q in place, write the
    rotated k and v to the rows' paged cache slots. positions int32 [rows], block_table int32
    [rows][stride]; kcache/vcache [num_blocks][block_size][kv_dim] of one layer."""
    rows = positions.numel()
    if qkv.shape[-1] != (head_num + 2 * kv_head_num) * head_size:
        raise ValueError(f"qkv rows of {qkv.shape[-1]} values, expected q, k and v exactly")
    _check_paged(qkv, qkv.shape[-1], head_num, kv_head_num, head_size, positions, block_table,
                 block_size, kcache, vcache)
    _call("sq8_paged_rope_kv", _ptr(qkv), rows, head_num, kv_head_num, head_size, _ptr(positions),
          _ptr(block_table), block_table.shape[-1], block_size, _ptr(sin_cache), _ptr(cos_cache),
          _ptr(kcache), _ptr(vcache), stream=stream)


def paged_attention_workspace_bytes(rows: int, head_num: int, kv_head_num: int, head_size: int,
                                    table_stride: int, block_size: int) -> int:
    """Bytes of the split-KV workspace for this shape (0: the kernel never splits it)."""
    return int(lib().sq8_paged_attention_workspace_bytes(rows, head_num, kv_head_num, head_size,
                                                         table_stride, block_size))


def paged_attention(qkv, q_stride: int, head_num: int, kv_head_num: int, head_size: int,
                    positions, block_table, block_size: int, kcache, vcache, out, workspace=None,
                    stream=None):
    """out[r] = attention of row r's query heads over positions 0..positions[r] of its sequence.
    With a workspace (zero-filled before its first use, of at least
    paged_attention_workspace_bytes() bytes) long rows split over several workgroups."""
    rows = positions.numel()
    _check_paged(qkv, q_stride, head_num, kv_head_num, head_size, positions, block_table,
                 block_size, kcache, vcache, out)
    if workspace is None:
        _call("sq8_paged_attention", _ptr(qkv), q_stride, rows, head_num, kv_head_num, head_size,
              _ptr(positions), _ptr(block_table), block_table.shape[-1], block_size,
              _ptr(kcache), _ptr(vcache), _ptr(out), stream=stream)
    else:
        _call("sq8_paged_attention_ws", _ptr(qkv), q_stride, rows, head_num, kv_head_num,
              head_size, _ptr(positions), _ptr(block_table), block_table.shape[-1], block_size,
              _ptr(kcache), _ptr(vcache), _ptr(out), _ptr(workspace),
              workspace.numel() * workspace.element_size(), stream=stream)


def swiglu_rows(gate_up, out, stream=None):
    """out[r][i] = silu(gate_up[r][i]) * gate_up[r][ffn + i]."""
    rows, two_ffn = gate_up.shape
    _call("sq8_swiglu_rows", _ptr(gate_up), rows, two_ffn // 2, _ptr(out), stream=stream)


def argmax_rows(logits, out, stream=None):
    """out[r] = first maximum of logits[r] (int32 on the device)."""
    rows, n = logits.shape
    _call("sq8_argmax_rows", _ptr(logits), rows, n, _ptr(out), stream=stream)
