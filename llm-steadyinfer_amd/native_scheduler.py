"""ctypes binding of the native continuous-batching scheduler (scheduler::Scheduler in
libsq8_op.so, src/source/scheduler/scheduler.cpp's interface; C entry points in
cpp/include/scheduler/scheduler_c.h).

NativeScheduler takes the same arguments and exposes the same results as scheduler.Scheduler, and
makes the same decisions step for step; the batching bookkeeping runs in C++ and calls the model
back once per step. A model with ``forward_arrays(tokens, positions, tables, num_decode)`` (numpy
int32 arrays; PagedBatchModel has it) gets the step's rows as arrays; otherwise it is called as
``forward(rows, tables)`` with row objects like scheduler.BatchRow.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Iterable, List, Optional

import numpy as np

from . import PKG_DIR

OP_LIB_PATH = PKG_DIR / "libsq8_op.so"
SCHED_SYMBOLS = ("sq8_sched_create", "sq8_sched_destroy", "sq8_sched_set_stop_tokens",
                 "sq8_sched_add_request", "sq8_sched_step", "sq8_sched_run",
                 "sq8_sched_all_finished", "sq8_sched_stats", "sq8_sched_generated",
                 "sq8_sched_finished_ids", "sq8_sched_last_rows", "sq8_sched_block_ref",
                 "sq8_sched_invariant", "sq8_sched_timing", "sq8_sched_batch_reconstruct_times",
                 "sq8_sched_kv_snapshot")
SQ8_SCHED_OK, SQ8_SCHED_ERR_ARG, SQ8_SCHED_ERR_MODEL, SQ8_SCHED_ERR_STEPS = 0, -1, -2, -3

_P32 = ctypes.POINTER(ctypes.c_int32)
FORWARD_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _P32,
                              _P32, _P32, _P32, ctypes.c_int, _P32)
_lib = None


def op_lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not OP_LIB_PATH.exists():
            raise RuntimeError(f"C++ op library not built: {OP_LIB_PATH} "
                               "(run __graft_entry__.build())")
        L = ctypes.CDLL(str(OP_LIB_PATH))
        vp, I = ctypes.c_void_p, ctypes.c_int
        L.sq8_sched_create.argtypes = [I, I, I, I, I, I, FORWARD_FN, vp]
        L.sq8_sched_create.restype = vp
        L.sq8_sched_destroy.argtypes = [vp]
        L.sq8_sched_destroy.restype = None
        L.sq8_sched_set_stop_tokens.argtypes = [vp, _P32, I]
        L.sq8_sched_add_request.argtypes = [vp, _P32, I]
        L.sq8_sched_step.argtypes = [vp]
        L.sq8_sched_run.argtypes = [vp, I]
        L.sq8_sched_all_finished.argtypes = [vp]
        L.sq8_sched_stats.argtypes = [vp, ctypes.POINTER(ctypes.c_int64), I]
        L.sq8_sched_generated.argtypes = [vp, I, _P32, I]
        L.sq8_sched_finished_ids.argtypes = [vp, _P32, I]
        L.sq8_sched_last_rows.argtypes = [vp, _P32, I]
        L.sq8_sched_block_ref.argtypes = [vp, I]
        L.sq8_sched_invariant.argtypes = [vp]
        PD = ctypes.POINTER(ctypes.c_double)
        L.sq8_sched_timing.argtypes = [vp, I, PD, PD, I]
        L.sq8_sched_batch_reconstruct_times.argtypes = [vp, PD, I]
        L.sq8_sched_kv_snapshot.argtypes = [vp, ctypes.POINTER(ctypes.c_int64), I]
        for name in SCHED_SYMBOLS:
            if name not in ("sq8_sched_create", "sq8_sched_destroy"):
                getattr(L, name).restype = I
        _lib = L
    return _lib


def _i32(a) -> "ctypes.Array":
    a = np.ascontiguousarray(a, dtype=np.int32)
    return a, a.ctypes.data_as(_P32)


@dataclass
class SeqRef:
    id: int


@dataclass
class Row:
    """One batch row handed to a row-based forward (the fields of scheduler.BatchRow)."""
    seq: SeqRef
    is_decode: bool
    token: int
    position: int


@dataclass
class FinishedSequence:
    """A finished request; times in seconds on the scheduler's clock (its creation is 0), as
    scheduler.Sequence's are on time.perf_counter()."""
    id: int
    prompt_tokens: List[int]
    generated_tokens: List[int] = field(default_factory=list)
    arrival_time: float = 0.0
    admit_time: float = 0.0
    first_token_time: float = 0.0
    last_token_time: float = 0.0
    finish_time: float = 0.0
    token_timestamps_ms: List[float] = field(default_factory=list)


class NativeScheduler:
    def __init__(self, forward, max_batch: int, max_seq_len: int, max_gen_len: int = 0,
                 block_size: int = 16, num_blocks: Optional[int] = None,
                 prefix_cache: bool = False, stop_tokens: Iterable[int] = ()):
        L = op_lib()
        self.forward = forward
        self.max_batch, self.max_seq_len, self.block_size = max_batch, max_seq_len, block_size
        self.max_blocks_per_seq = (max_seq_len + block_size - 1) // block_size
        self._error = None
        native = getattr(forward, "native_forward", None)
        if native is not None:  # a native model: C++ calls C++, no Python in the step loop
            self._cb = FORWARD_FN(native[0])
            user = native[1]
        else:
            self._cb = FORWARD_FN(self._forward)  # kept alive as long as the handle
            user = None
        self._native = native is not None
        self._h = L.sq8_sched_create(max_batch, max_seq_len, max_gen_len, block_size,
                                     num_blocks or 0, int(bool(prefix_cache)), self._cb, user)
        if not self._h:
            raise ValueError("bad scheduler arguments")
        stop, p = _i32(list(stop_tokens))
        self._check(L.sq8_sched_set_stop_tokens(self._h, p, len(stop)))
        self._prompts = {}

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            op_lib().sq8_sched_destroy(h)
            self._h = None

    @staticmethod
    def _check(rc):
        if rc < 0:
            raise RuntimeError(f"native scheduler status {rc}")
        return rc

    # ------------------------------------------------------------------ the model callback
    def _forward(self, _user, batch, nd, tok_p, pos_p, ids_p, tab_p, stride, next_p):
        try:
            tok = np.ctypeslib.as_array(tok_p, (batch,)).copy()
            pos = np.ctypeslib.as_array(pos_p, (batch,)).copy()
            tab = np.ctypeslib.as_array(tab_p, (batch, stride)).copy()
            if hasattr(self.forward, "forward_arrays"):
                out = self.forward.forward_arrays(tok, pos, tab, nd)
            else:
                ids = np.ctypeslib.as_array(ids_p, (batch,))
                rows = [Row(SeqRef(int(ids[i])), i < nd, int(tok[i]), int(pos[i]))
                        for i in range(batch)]
                out = self.forward(rows, tab.tolist())
            if len(out) != nd:
                raise RuntimeError(f"forward returned {len(out)} tokens for {nd} decode rows")
            if nd:
                np.ctypeslib.as_array(next_p, (nd,))[:] = np.asarray(out, dtype=np.int32)
            return 0
        except BaseException as e:  # noqa: BLE001 - reported by step()
            self._error = e
            return 1

    # ------------------------------------------------------------------ Scheduler interface
    def add_request(self, prompt: List[int]) -> int:
        arr, p = _i32(list(prompt))
        sid = op_lib().sq8_sched_add_request(self._h, p, len(arr))
        if sid >= 0:
            self._prompts[sid] = [int(t) for t in prompt]
        return sid

    def _raise_model_error(self):
        if self._error is not None:
            e, self._error = self._error, None
            raise e
        if self._native:
            raise RuntimeError("native model: " + self.forward.last_error())
        raise RuntimeError("model forward failed")

    def step(self) -> None:
        rc = op_lib().sq8_sched_step(self._h)
        if rc == SQ8_SCHED_ERR_MODEL:
            self._raise_model_error()
        self._check(rc)

    def all_finished(self) -> bool:
        return bool(self._check(op_lib().sq8_sched_all_finished(self._h)))

    def run(self, max_steps: Optional[int] = None) -> List[FinishedSequence]:
        """Step until every request finished (RuntimeError after max_steps steps). With a native
        model the whole loop runs in C++ (sq8_sched_run)."""
        if self._native:
            rc = op_lib().sq8_sched_run(self._h, max_steps or 0)
            if rc == SQ8_SCHED_ERR_STEPS:
                raise RuntimeError(f"scheduler made no progress within {max_steps} steps")
            if rc == SQ8_SCHED_ERR_MODEL:
                self._raise_model_error()
            self._check(rc)
            return sorted(self.finished, key=lambda q: q.id)
        while not self.all_finished():
            if max_steps is not None and self.steps >= max_steps:
                raise RuntimeError(f"scheduler made no progress within {max_steps} steps")
            self.step()
        return sorted(self.finished, key=lambda s: s.id)

    def _stats(self):
        out = (ctypes.c_int64 * 10)()
        self._check(op_lib().sq8_sched_stats(self._h, out, 10))
        return list(out)

    @property
    def steps(self) -> int:
        return self._stats()[0]

    @property
    def rows_run(self) -> int:
        return self._stats()[1]

    @property
    def preemptions(self) -> int:
        return self._stats()[2]

    @property
    def shared_prefix_blocks(self) -> int:
        return self._stats()[3]

    @property
    def prefill_budget(self) -> int:
        return self._stats()[7]

    def free_block_count(self) -> int:
        return self._stats()[8]

    def prefix_entries(self) -> int:
        return self._stats()[9]

    def generated(self, seq_id: int) -> List[int]:
        L = op_lib()
        n = self._check(L.sq8_sched_generated(self._h, seq_id, None, 0))
        buf = (ctypes.c_int32 * max(n, 1))()
        L.sq8_sched_generated(self._h, seq_id, buf, n)
        return list(buf[:n])

    @property
    def finished(self) -> List[FinishedSequence]:
        L = op_lib()
        n = self._check(L.sq8_sched_finished_ids(self._h, None, 0))
        buf = (ctypes.c_int32 * max(n, 1))()
        L.sq8_sched_finished_ids(self._h, buf, n)
        return [self._finished(i) for i in buf[:n]]

    def _finished(self, i: int) -> FinishedSequence:
        L = op_lib()
        times = (ctypes.c_double * 5)()
        n = self._check(L.sq8_sched_timing(self._h, i, times, None, 0))
        itl = (ctypes.c_double * max(n, 1))()
        L.sq8_sched_timing(self._h, i, times, itl, n)
        t = [v / 1e3 for v in times]
        return FinishedSequence(i, self._prompts[i], self.generated(i), *t, list(itl[:n]))

    @property
    def batch_reconstruct_times_ms(self) -> List[float]:
        L = op_lib()
        n = self._check(L.sq8_sched_batch_reconstruct_times(self._h, None, 0))
        buf = (ctypes.c_double * max(n, 1))()
        L.sq8_sched_batch_reconstruct_times(self._h, buf, n)
        return list(buf[:n])

    def last_rows(self):
        """(seq id, is_decode, token, position) of each row of the last step."""
        L = op_lib()
        n = self._check(L.sq8_sched_last_rows(self._h, None, 0))
        buf = (ctypes.c_int32 * max(4 * n, 1))()
        L.sq8_sched_last_rows(self._h, buf, n)
        return [tuple(buf[4 * i:4 * i + 4]) for i in range(n)]

    def kv_snapshot(self):
        """(busy KV rows, tokens held by the running sequences, tokens of KV allocated)."""
        out = (ctypes.c_int64 * 3)()
        self._check(op_lib().sq8_sched_kv_snapshot(self._h, out, 3))
        return tuple(out)

    def block_ref(self, block: int) -> int:
        return self._check(op_lib().sq8_sched_block_ref(self._h, block))

    def invariant_holds(self) -> bool:
        return bool(self._check(op_lib().sq8_sched_invariant(self._h)))


class NativePagedBatchModel:
    """model::PagedBatchModel (C++, libsq8_op.so) over the weights dict of
    batch_model.PagedBatchModel (device tensors: "qkv", "o", "gu", "down" lists of (q, s) per
    layer, "cls" (q, s), "emb", "norm" list of 2 L + 1). The same launches in the same order as
    the Python model, from C++, on the model's own stream. With packed the projections are
    repacked once (sq8_pack_weights) and the model holds the packed copies.

    Handed to NativeScheduler, the scheduler calls it directly (native_forward); with the Python
    scheduler, forward / forward_arrays go through ctypes."""

    def __init__(self, cfg, weights: dict, group_size: int, max_rows: int, max_seq_len: int,
                 num_blocks: int, block_size: int, device="cuda", use_graphs: bool = True,
                 split_kv: bool = True, packed: bool = False, eps: float = 1e-6):
        import torch
        from . import pack_weights
        L = op_lib()
        _bind_model(L)
        self.torch = torch
        if packed:
            weights = dict(weights)
            for key in ("qkv", "o", "gu", "down"):
                weights[key] = [(pack_weights(q), s) for q, s in weights[key]]
            weights["cls"] = (pack_weights(weights["cls"][0]), weights["cls"][1])
        self.w = weights  # the model reads these device buffers for its lifetime
        self.max_rows, self.block_size = max_rows, block_size
        self.max_blocks_per_seq = (max_seq_len + block_size - 1) // block_size
        nl = cfg.layer_num
        ptrs = lambda ts, T: (T * len(ts))(*[t.data_ptr() for t in ts])
        P8, PF = ctypes.c_void_p, ctypes.c_void_p
        c = ModelConfigC(cfg.dim, cfg.hidden_dim, nl, cfg.head_num, cfg.kv_head_num, cfg.vocab,
                         float(cfg.rope_theta), group_size, eps)
        arrs = {k: (ptrs([q for q, _ in weights[k]], P8), ptrs([s for _, s in weights[k]], PF))
                for k in ("qkv", "o", "gu", "down")}
        norm = ptrs(weights["norm"], PF)
        err = ctypes.c_char_p()
        self._h = L.sq8_batch_model_create(
            ctypes.byref(c), arrs["qkv"][0], arrs["qkv"][1], arrs["o"][0], arrs["o"][1],
            arrs["gu"][0], arrs["gu"][1], arrs["down"][0], arrs["down"][1],
            weights["cls"][0].data_ptr(), weights["cls"][1].data_ptr(),
            weights["emb"].data_ptr(), norm, int(packed), max_rows, max_seq_len, num_blocks,
            block_size, int(use_graphs), int(split_kv), None, ctypes.byref(err))
        if not self._h:
            raise RuntimeError("native batch model: " + (err.value or b"?").decode())
        self.native_forward = (ctypes.cast(L.sq8_batch_model_forward, ctypes.c_void_p).value,
                               self._h)

    @classmethod
    def from_file(cls, path, max_rows: int, max_seq_len: int, num_blocks: int, block_size: int,
                  use_graphs: bool = True, split_kv: bool = True, packed: bool = False):
        """The model from an INT8 model file, read and uploaded in C++ (model::Int8ModelFile,
        model::DeviceWeights); no Python touches the weights."""
        L = op_lib()
        _bind_model(L)
        self = cls.__new__(cls)
        self.w = None
        self.max_rows, self.block_size = max_rows, block_size
        self.max_blocks_per_seq = (max_seq_len + block_size - 1) // block_size
        err = ctypes.c_char_p()
        self._h = L.sq8_batch_model_create_from_file(
            str(path).encode(), int(packed), max_rows, max_seq_len, num_blocks, block_size,
            int(use_graphs), int(split_kv), ctypes.byref(err))
        if not self._h:
            raise RuntimeError("native batch model: " + (err.value or b"?").decode())
        self.native_forward = (ctypes.cast(L.sq8_batch_model_forward, ctypes.c_void_p).value,
                               self._h)
        return self

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            op_lib().sq8_batch_model_destroy(h)
            self._h = None

    def last_error(self) -> str:
        return op_lib().sq8_batch_model_last_error(self._h).decode()

    def capture_decode_graphs(self) -> float:
        import time
        t0 = time.perf_counter()
        if op_lib().sq8_batch_model_capture_decode_graphs(self._h):
            raise RuntimeError("native batch model: " + self.last_error())
        return time.perf_counter() - t0

    def _stats(self):
        out = (ctypes.c_int64 * 3)()
        op_lib().sq8_batch_model_stats(self._h, out, 3)
        return list(out)

    @property
    def graph_replays(self) -> int:
        return self._stats()[0]

    @property
    def rows_run(self) -> int:
        return self._stats()[1]

    @property
    def graphs(self):
        return range(self._stats()[2])

    def forward_arrays(self, tok, pos, tab, nd: int):
        tok, tp = _i32(tok)
        pos, pp = _i32(pos)
        tab, bp = _i32(tab)
        B = len(tok)
        out = (ctypes.c_int32 * max(nd, 1))()
        if op_lib().sq8_batch_model_forward(self._h, B, nd, tp, pp, None, bp, tab.shape[1], out):
            raise RuntimeError("native batch model: " + self.last_error())
        return list(out[:nd])

    def forward(self, rows, tables):
        nd = sum(1 for r in rows if r.is_decode)
        return self.forward_arrays([r.token for r in rows], [r.position for r in rows],
                                   np.asarray(tables, np.int32).reshape(len(rows), -1), nd)


class NativeInt8Decoder:
    """model::Int8Decoder (C++, libsq8_op.so): the greedy single-sequence decoder of decoder.py
    (fused step, one HIP-graph replay per token) over the same weight dict (row-major)."""

    def __init__(self, cfg, weights: dict, group_size: int, max_seq: int,
                 split_attention: bool = True, eps: float = 1e-6):
        L = op_lib()
        _bind_model(L)
        self.w, self.cfg, self.max_seq = weights, cfg, max_seq
        ptrs = lambda ts: (ctypes.c_void_p * len(ts))(*[t.data_ptr() for t in ts])
        c = ModelConfigC(cfg.dim, cfg.hidden_dim, cfg.layer_num, cfg.head_num, cfg.kv_head_num,
                         cfg.vocab, float(cfg.rope_theta), group_size, eps)
        arrs = {k: (ptrs([q for q, _ in weights[k]]), ptrs([s for _, s in weights[k]]))
                for k in ("qkv", "o", "gu", "down")}
        err = ctypes.c_char_p()
        self._h = L.sq8_decoder_create(
            ctypes.byref(c), arrs["qkv"][0], arrs["qkv"][1], arrs["o"][0], arrs["o"][1],
            arrs["gu"][0], arrs["gu"][1], arrs["down"][0], arrs["down"][1],
            weights["cls"][0].data_ptr(), weights["cls"][1].data_ptr(),
            weights["emb"].data_ptr(), ptrs(weights["norm"]), max_seq, int(split_attention),
            None, ctypes.byref(err))
        if not self._h:
            raise RuntimeError("native decoder: " + (err.value or b"?").decode())

    @classmethod
    def from_file(cls, path, max_seq: int, split_attention: bool = True):
        """The decoder from an INT8 model file, read and uploaded in C++."""
        L = op_lib()
        _bind_model(L)
        self = cls.__new__(cls)
        self.w, self.cfg, self.max_seq = None, None, max_seq
        err = ctypes.c_char_p()
        self._h = L.sq8_decoder_create_from_file(str(path).encode(), max_seq,
                                                 int(split_attention), ctypes.byref(err))
        if not self._h:
            raise RuntimeError("native decoder: " + (err.value or b"?").decode())
        return self

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            op_lib().sq8_decoder_destroy(h)
            self._h = None

    def generate(self, prompt, n_new: int, use_graph: bool = True):
        arr, p = _i32(list(prompt))
        out = (ctypes.c_int32 * max(n_new, 1))()
        if op_lib().sq8_decoder_generate(self._h, p, len(arr), n_new, out, int(use_graph)):
            raise RuntimeError("native decoder: " +
                               op_lib().sq8_decoder_last_error(self._h).decode())
        return list(out[:n_new])


class ModelConfigC(ctypes.Structure):
    _fields_ = [("dim", ctypes.c_int), ("hidden_dim", ctypes.c_int),
                ("layer_num", ctypes.c_int), ("head_num", ctypes.c_int),
                ("kv_head_num", ctypes.c_int), ("vocab_size", ctypes.c_int),
                ("rope_theta", ctypes.c_float), ("group_size", ctypes.c_int),
                ("eps", ctypes.c_float)]


MODEL_SYMBOLS = ("sq8_batch_model_create", "sq8_batch_model_destroy", "sq8_batch_model_forward",
                 "sq8_batch_model_capture_decode_graphs", "sq8_batch_model_stats",
                 "sq8_batch_model_last_error", "sq8_decoder_create", "sq8_decoder_destroy",
                 "sq8_decoder_generate", "sq8_decoder_last_error",
                 "sq8_batch_model_create_from_file", "sq8_decoder_create_from_file")
_model_bound = False


def _bind_model(L):
    global _model_bound
    if _model_bound:
        return
    vp, I = ctypes.c_void_p, ctypes.c_int
    L.sq8_batch_model_create.argtypes = [ctypes.POINTER(ModelConfigC)] + [vp] * 12 + \
        [I, I, I, I, I, I, I, vp, ctypes.POINTER(ctypes.c_char_p)]
    L.sq8_batch_model_create.restype = vp
    L.sq8_batch_model_destroy.argtypes = [vp]
    L.sq8_batch_model_destroy.restype = None
    L.sq8_batch_model_forward.argtypes = [vp, I, I, _P32, _P32, _P32, _P32, I, _P32]
    L.sq8_batch_model_forward.restype = I
    L.sq8_batch_model_capture_decode_graphs.argtypes = [vp]
    L.sq8_batch_model_capture_decode_graphs.restype = I
    L.sq8_batch_model_stats.argtypes = [vp, ctypes.POINTER(ctypes.c_int64), I]
    L.sq8_batch_model_stats.restype = I
    L.sq8_batch_model_last_error.argtypes = [vp]
    L.sq8_batch_model_last_error.restype = ctypes.c_char_p
    L.sq8_decoder_create.argtypes = [ctypes.POINTER(ModelConfigC)] + [vp] * 12 + \
        [I, I, vp, ctypes.POINTER(ctypes.c_char_p)]
    L.sq8_decoder_create.restype = vp
    L.sq8_decoder_destroy.argtypes = [vp]
    L.sq8_decoder_destroy.restype = None
    L.sq8_decoder_generate.argtypes = [vp, _P32, I, I, _P32, I]
    L.sq8_decoder_generate.restype = I
    L.sq8_decoder_last_error.argtypes = [vp]
    L.sq8_decoder_last_error.restype = ctypes.c_char_p
    L.sq8_batch_model_create_from_file.argtypes = [ctypes.c_char_p, I, I, I, I, I, I, I,
                                                   ctypes.POINTER(ctypes.c_char_p)]
    L.sq8_batch_model_create_from_file.restype = vp
    L.sq8_decoder_create_from_file.argtypes = [ctypes.c_char_p, I, I,
                                               ctypes.POINTER(ctypes.c_char_p)]
    L.sq8_decoder_create_from_file.restype = vp
    _model_bound = True
