"""INT8 model file (``.bin``) of LLM-SteadyInfer: layout, random-init writer and memory-mapped reader.

The reference loads, but does not ship a writer for, this format:
- header: ``ModelConfig`` (src/include/model/config.h:4-14): eight int32 (dim, hidden_dim,
  layer_num, head_num, kv_head_num, vocab_size, seq_len, immediate_dim) and one float
  (rope_theta), 36 bytes, little endian;
- then ``int32 group_size`` for quantised files (src/source/model/model.cpp:305-311);
- then the weights, consumed by a byte cursor in this order (llama3.cpp:193-297; qwen2.cpp:193-297
  is the same): wq x L, wk x L, wv x L, wo x L, w1 x L, w2 x L, w3 x L, the classifier (only when
  the header's vocab_size is negative), then fp32 data: the token embedding [|vocab|, dim] and
  2L + 1 RMSNorm weights [dim] (attention, ffn, final).
- every quantised matrix [rows, cols] is int8 row-major followed by its rows*cols/group_size fp32
  scales (LayerParam::set_weight, src/source/op/layer.cpp:184-218).
- the sign of vocab_size selects tied weights (Model::generate_model_infos, model.cpp:369-373):
  vocab_size > 0 means "shared": the loader then binds the int8 classifier at the cursor that is
  also the start of the fp32 embedding and does not advance (llama3.cpp:268-277). Real tied files
  are therefore not self-consistent; the writer emits untied files (negative vocab_size) by
  default, and the reader reproduces the reference's cursor for either sign.

The quantiser is the benchmark's group-wise symmetric absmax quantiser: s = absmax/127 (fp32),
q = round-half-away-from-zero(w / s) clamped to +-127, zero group -> s = 0, q = 0.
"""
from __future__ import annotations

import dataclasses
import struct
from pathlib import Path

import numpy as np

HEADER_FMT = "<8if"                      # ModelConfig, config.h:4-14
HEADER_BYTES = struct.calcsize(HEADER_FMT)  # 36
GROUP_FMT = "<i"                         # int32 group_size, model.cpp:305-311
QUANT_ORDER = ("wq", "wk", "wv", "wo", "w1", "w2", "w3")


@dataclasses.dataclass
class ModelConfig:
    """Header fields in file order (config.h:4-14)."""
    dim: int
    hidden_dim: int
    layer_num: int
    head_num: int
    kv_head_num: int
    vocab_size: int          # > 0: tied classifier, < 0: untied (model.cpp:369-373)
    seq_len: int
    immediate_dim: int = 0
    rope_theta: float = 1000000.0

    @property
    def kv_dim(self) -> int:
        """model.cpp:363."""
        return (self.dim * self.kv_head_num) // self.head_num

    @property
    def vocab(self) -> int:
        return abs(self.vocab_size)

    @property
    def shared(self) -> bool:
        return self.vocab_size > 0

    def pack(self) -> bytes:
        return struct.pack(HEADER_FMT, self.dim, self.hidden_dim, self.layer_num, self.head_num,
                           self.kv_head_num, self.vocab_size, self.seq_len, self.immediate_dim,
                           self.rope_theta)

    @classmethod
    def unpack(cls, raw: bytes) -> "ModelConfig":
        return cls(*struct.unpack(HEADER_FMT, raw[:HEADER_BYTES]))


# Llama-3-8B and Qwen2-1.5B shapes of the benchmark configs (untied, so the writer's files load).
LLAMA3_8B = ModelConfig(dim=4096, hidden_dim=14336, layer_num=32, head_num=32, kv_head_num=8,
                        vocab_size=-128256, seq_len=8192, rope_theta=500000.0)
QWEN2_1_5B = ModelConfig(dim=1536, hidden_dim=8960, layer_num=28, head_num=12, kv_head_num=2,
                         vocab_size=-151936, seq_len=8192, rope_theta=1000000.0)


@dataclasses.dataclass(frozen=True)
class Entry:
    """One tensor of the file: ``offset`` is from the start of the weights (after the group size).
    Quantised entries have ``scale_offset`` (the trailing fp32 block); fp32 entries have None."""
    name: str
    layer: int
    rows: int
    cols: int
    offset: int
    scale_offset: int | None

    @property
    def quantised(self) -> bool:
        return self.scale_offset is not None


def quant_shapes(cfg: ModelConfig) -> dict:
    """[rows, cols] of each quantised projection (llama3.cpp:201-263)."""
    d, h, kv = cfg.dim, cfg.hidden_dim, cfg.kv_dim
    return {"wq": (d, d), "wk": (kv, d), "wv": (kv, d), "wo": (d, d),
            "w1": (h, d), "w2": (d, h), "w3": (h, d)}


def layout(cfg: ModelConfig, group_size: int) -> list:
    """Every tensor with its byte offset, following the reference's cursor arithmetic
    (``pos += rows*cols + scale_num*sizeof(float)``, llama3.cpp:206-277; then fp32 pointers,
    llama3.cpp:280-296)."""
    shapes = quant_shapes(cfg)
    out = []
    pos = 0
    for name in QUANT_ORDER:
        rows, cols = shapes[name]
        if (rows * cols) % group_size:
            raise ValueError(f"{name}: {rows}x{cols} not a multiple of group size {group_size}")
        for i in range(cfg.layer_num):
            out.append(Entry(name, i, rows, cols, pos, pos + rows * cols))
            pos += rows * cols + (rows * cols // group_size) * 4
    cls_rows = cfg.vocab
    out.append(Entry("cls", 0, cls_rows, cfg.dim, pos, pos + cls_rows * cfg.dim))
    if not cfg.shared:
        pos += cls_rows * cfg.dim + (cls_rows * cfg.dim // group_size) * 4
    out.append(Entry("embedding", 0, cfg.vocab, cfg.dim, pos, None))
    pos += cfg.vocab * cfg.dim * 4
    for i in range(2 * cfg.layer_num + 1):
        out.append(Entry("rmsnorm", i, 1, cfg.dim, pos, None))
        pos += cfg.dim * 4
    return out


def file_bytes(cfg: ModelConfig, group_size: int) -> int:
    e = layout(cfg, group_size)[-1]
    return HEADER_BYTES + 4 + e.offset + e.cols * 4


def quantize(w: np.ndarray, group_size: int):
    """Group absmax quantiser over the flat array: returns (q int8, scales fp32 [numel/gs])."""
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1, group_size)
    amax = np.max(np.abs(w), axis=1)
    s = (amax / np.float32(127.0)).astype(np.float32)
    safe = np.where(s == 0, np.float32(1.0), s)       # an all-zero group quantises to 0
    v = w / safe[:, None]                              # the fp32 quotient
    # |v| + 0.5 is exact in fp32 for |v| <= 127.5, so this is round-half-away-from-zero.
    r = np.minimum(np.floor(np.abs(v) + np.float32(0.5)), np.float32(127.0))
    return np.copysign(r, v).astype(np.int8).reshape(-1), s


def _block_rng(seed: int, name: str, layer: int) -> np.random.Generator:
    tag = QUANT_ORDER.index(name) if name in QUANT_ORDER else 16 + ("cls", "embedding",
                                                                     "rmsnorm").index(name)
    return np.random.default_rng([seed, tag, layer])


def _row_step(rows: int, cols: int, group_size: int, rows_per_chunk: int) -> int:
    """Rows per written chunk: a chunk must hold whole groups (groups may span rows)."""
    align = group_size // np.gcd(cols, group_size)
    return max(align, (min(rows, rows_per_chunk) // align) * align)


def _random_blocks(cfg: ModelConfig, group_size: int, seed: int, w_std: float,
                   rows_per_chunk: int):
    """The random-init tensors in file order, in row chunks: yields (entry, first row, q, s) for
    quantised chunks and (entry, first row, fp32 rows, None) for fp32 ones. Projection weights
    ~ N(0, w_std) quantised per group, embedding ~ N(0, 1), RMSNorm weights 1; each tensor has
    its own generator, so the values do not depend on how they are consumed."""
    for e in layout(cfg, group_size):
        rng = _block_rng(seed, e.name, e.layer)
        if e.quantised:
            if e.name == "cls" and cfg.shared:
                continue  # the tied classifier has no bytes of its own (reference quirk)
            step = _row_step(e.rows, e.cols, group_size, rows_per_chunk)
            for r0 in range(0, e.rows, step):
                r1 = min(e.rows, r0 + step)
                wchunk = (rng.standard_normal((r1 - r0, e.cols), dtype=np.float32)
                          * np.float32(w_std))
                q, sc = quantize(wchunk, group_size)
                yield e, r0, q, sc
        elif e.name == "embedding":
            for r0 in range(0, e.rows, rows_per_chunk):
                r1 = min(e.rows, r0 + rows_per_chunk)
                yield e, r0, rng.standard_normal((r1 - r0, e.cols), dtype=np.float32), None
        else:
            yield e, 0, np.ones((1, e.cols), np.float32), None


def write_random(path, cfg: ModelConfig, group_size: int = 64, seed: int = 0,
                 w_std: float = 0.02, rows_per_chunk: int = 4096) -> Path:
    """Write a random-init INT8 model file: projection weights ~ N(0, w_std) quantised per group,
    embedding ~ N(0, 1), RMSNorm weights 1. Streams row chunks, so memory stays bounded for the
    Llama-3-8B shapes. Deterministic in ``seed``."""
    path = Path(path)
    base = HEADER_BYTES + 4
    with open(path, "wb") as f:
        f.write(cfg.pack())
        f.write(struct.pack(GROUP_FMT, group_size))
        f.truncate(file_bytes(cfg, group_size))
        for e, r0, a, sc in _random_blocks(cfg, group_size, seed, w_std, rows_per_chunk):
            if sc is not None:
                f.seek(base + e.offset + r0 * e.cols)
                f.write(a.tobytes())
                f.seek(base + e.scale_offset + (r0 * e.cols // group_size) * 4)
                f.write(sc.tobytes())
            else:
                f.seek(base + e.offset + r0 * e.cols * 4)
                f.write(a.tobytes())
    return path


class RandomModel:
    """The model ``write_random`` would write with the same arguments, held in host memory with
    ModelFile's accessors (config, group_size, quant, fp32): for tests and benchmarks at full
    widths without the file round trip. Bit-identical to reading the written file."""

    def __init__(self, cfg: ModelConfig, group_size: int = 64, seed: int = 0,
                 w_std: float = 0.02, rows_per_chunk: int = 4096):
        self.config, self.group_size = cfg, group_size
        self._q, self._f = {}, {}
        for e, r0, a, sc in _random_blocks(cfg, group_size, seed, w_std, rows_per_chunk):
            key = (e.name, e.layer)
            if sc is not None:
                if key not in self._q:
                    self._q[key] = (np.empty((e.rows, e.cols), np.int8),
                                    np.empty(e.rows * e.cols // group_size, np.float32))
                q, s = self._q[key]
                q.reshape(-1)[r0 * e.cols:r0 * e.cols + a.size] = a
                s0 = r0 * e.cols // group_size
                s[s0:s0 + sc.size] = sc
            else:
                if key not in self._f:
                    self._f[key] = np.empty((e.rows, e.cols), np.float32)
                self._f[key][r0:r0 + a.shape[0]] = a
        if cfg.shared:  # the reference binds the tied classifier at the embedding's bytes
            raise ValueError("RandomModel holds untied models only (negative vocab_size)")

    def quant(self, name: str, layer: int = 0):
        return self._q[(name, layer)]

    def fp32(self, name: str, layer: int = 0) -> np.ndarray:
        return self._f[(name, layer)]


def regenerate_block(cfg: ModelConfig, group_size: int, name: str, layer: int, seed: int = 0,
                     w_std: float = 0.02, rows_per_chunk: int = 4096) -> np.ndarray:
    """The fp32 weights ``write_random`` quantised for one projection (for checks)."""
    rows, cols = (cfg.vocab, cfg.dim) if name == "cls" else quant_shapes(cfg)[name]
    rng = _block_rng(seed, name, layer)
    step = _row_step(rows, cols, group_size, rows_per_chunk)
    parts = [rng.standard_normal((min(rows, r0 + step) - r0, cols), dtype=np.float32)
             * np.float32(w_std) for r0 in range(0, rows, step)]
    return np.concatenate(parts, axis=0)


class ModelFile:
    """Memory-mapped reader with the reference's offsets (Model::read_model_file,
    model.cpp:295-353): ``quant(name, layer)`` returns (int8 [rows, cols], fp32 scales)."""

    def __init__(self, path):
        self.path = Path(path)
        self.raw = np.memmap(self.path, dtype=np.uint8, mode="r")
        if self.raw.size < HEADER_BYTES + 4:
            raise ValueError("file shorter than the header")
        self.config = ModelConfig.unpack(self.raw[:HEADER_BYTES].tobytes())
        self.group_size = struct.unpack(GROUP_FMT, self.raw[HEADER_BYTES:HEADER_BYTES + 4].tobytes())[0]
        if self.group_size <= 0:
            raise ValueError(f"bad group size {self.group_size}")
        self.base = HEADER_BYTES + 4
        self.entries = {(e.name, e.layer): e for e in layout(self.config, self.group_size)}
        need = file_bytes(self.config, self.group_size)
        if self.raw.size < need:
            raise ValueError(f"file has {self.raw.size} bytes, layout needs {need}")

    def quant(self, name: str, layer: int = 0):
        e = self.entries[(name, layer)]
        n = e.rows * e.cols
        q = self.raw[self.base + e.offset:self.base + e.offset + n].view(np.int8)
        s = self.raw[self.base + e.scale_offset:self.base + e.scale_offset
                     + (n // self.group_size) * 4].view(np.float32)
        return q.reshape(e.rows, e.cols), s

    def fp32(self, name: str, layer: int = 0) -> np.ndarray:
        e = self.entries[(name, layer)]
        n = e.rows * e.cols
        return self.raw[self.base + e.offset:self.base + e.offset + 4 * n].view(np.float32).reshape(
            e.rows, e.cols)
