"""INT8 model file: layout, random-init writer, Python reader and the C++ loader
(model/int8_model_file.h, exercised through tests/cpp/test_model_file.cpp)."""
import importlib
import struct
import subprocess

import numpy as np
import pytest

from conftest import REPO, load_pkg
from oracle import sq8_oracle as o

BIN = REPO / "llm-steadyinfer_amd" / "_build" / "test_model_file"
load_pkg()
mf = importlib.import_module("llm_steadyinfer_amd.model_file")

TINY = mf.ModelConfig(dim=128, hidden_dim=320, layer_num=2, head_num=4, kv_head_num=2,
                      vocab_size=-300, seq_len=64, rope_theta=500000.0)
TINY_TIED = mf.ModelConfig(dim=128, hidden_dim=320, layer_num=2, head_num=4, kv_head_num=2,
                           vocab_size=300, seq_len=64)


def _cpp(*args, timeout=60):
    if not BIN.exists():
        pytest.fail(f"{BIN} not built (run __graft_entry__.build())")
    res = subprocess.run([str(BIN), *map(str, args)], capture_output=True, text=True,
                         timeout=timeout)
    print(res.stdout[-3000:], res.stderr[-2000:])
    return res


def test_header_is_the_reference_struct():
    """36-byte ModelConfig (8 x int32 + float) then int32 group size."""
    assert mf.HEADER_BYTES == 36
    raw = TINY.pack()
    assert struct.unpack("<8if", raw) == (128, 320, 2, 4, 2, -300, 64, 0, 500000.0)
    assert mf.ModelConfig.unpack(raw) == TINY


def test_llama3_8b_layout_sizes():
    """Offsets follow the reference cursor: 7 projections x 32 layers, untied classifier, fp32
    embedding and 65 RMSNorm vectors; int8 bytes + N*K/16 scale bytes per projection."""
    cfg, gs = mf.LLAMA3_8B, 64
    ents = mf.layout(cfg, gs)
    per_layer = 2 * 4096 * 4096 + 2 * 1024 * 4096 + 3 * 14336 * 4096
    quant = 32 * per_layer + 128256 * 4096
    emb = next(e for e in ents if e.name == "embedding")
    assert emb.offset == quant * 17 // 16
    assert ents[-1].name == "rmsnorm" and ents[-1].layer == 64
    assert mf.file_bytes(cfg, gs) == 40 + quant * 17 // 16 + 128256 * 4096 * 4 + 65 * 4096 * 4
    w2 = [e for e in ents if e.name == "w2"]
    assert (w2[0].rows, w2[0].cols) == (4096, 14336)
    assert w2[1].offset - w2[0].offset == 4096 * 14336 * 17 // 16
    assert all(e.scale_offset == e.offset + e.rows * e.cols for e in ents if e.quantised)


def test_tied_layout_binds_classifier_at_the_embedding():
    """vocab_size > 0: the classifier cursor is not advanced (llama3.cpp:268-277)."""
    ents = {(e.name, e.layer): e for e in mf.layout(TINY_TIED, 64)}
    assert ents[("cls", 0)].offset == ents[("embedding", 0)].offset
    untied = {(e.name, e.layer): e for e in mf.layout(TINY, 64)}
    assert (untied[("embedding", 0)].offset - untied[("cls", 0)].offset
            == 300 * 128 * 17 // 16)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_writer_quantiser_is_the_oracle_quantiser(seed):
    """The product quantiser (numpy, fp32 quotient) equals the oracle's C quantiser bit for bit,
    including exact ties, zero groups and extreme magnitudes."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal(64 * 2000) * 10.0 ** rng.uniform(-6, 6, 64 * 2000)).astype(np.float32)
    w[:64] = 0
    w[64:128] = np.float32(127.5) * np.arange(64, dtype=np.float32) / 63
    w[128:192] = -w[64:128]
    q, s = mf.quantize(w, 64)
    q2, s2 = o.quantize(w, 64)
    np.testing.assert_array_equal(q, q2.reshape(-1))
    np.testing.assert_array_equal(s, s2)


@pytest.mark.parametrize("cfg,gs", [(TINY, 64), (TINY, 32), (TINY_TIED, 64)])
def test_write_then_read(tmp_path, cfg, gs):
    """Every projection read back equals the quantisation of the regenerated weights; fp32 tensors
    are the embedding and unit RMSNorm weights; the file has exactly the layout's size."""
    path = mf.write_random(tmp_path / "m.bin", cfg, gs, seed=7, rows_per_chunk=96)
    assert path.stat().st_size == mf.file_bytes(cfg, gs)
    m = mf.ModelFile(path)
    assert m.config == cfg and m.group_size == gs
    for name in mf.QUANT_ORDER:
        for layer in range(cfg.layer_num):
            q, s = m.quant(name, layer)
            w = mf.regenerate_block(cfg, gs, name, layer, seed=7, rows_per_chunk=96)
            q2, s2 = o.quantize(w, gs)
            np.testing.assert_array_equal(q, q2)
            np.testing.assert_array_equal(s, s2)
    if not cfg.shared:
        q, s = m.quant("cls")
        q2, s2 = o.quantize(mf.regenerate_block(cfg, gs, "cls", 0, seed=7, rows_per_chunk=96), gs)
        np.testing.assert_array_equal(q, q2)
    np.testing.assert_array_equal(m.fp32("rmsnorm", 2 * cfg.layer_num), np.ones((1, cfg.dim)))
    emb = m.fp32("embedding")
    assert emb.shape == (cfg.vocab, cfg.dim) and abs(float(emb.std()) - 1.0) < 0.05


@pytest.mark.parametrize("gs", [64, 32])
def test_random_model_equals_written_file(tmp_path, gs):
    """RandomModel (in memory) holds exactly the bytes write_random puts in the file."""
    path = mf.write_random(tmp_path / "m.bin", TINY, gs, seed=3, rows_per_chunk=96)
    m, r = mf.ModelFile(path), mf.RandomModel(TINY, gs, seed=3, rows_per_chunk=96)
    assert r.config == m.config and r.group_size == m.group_size
    for name in mf.QUANT_ORDER:
        for layer in range(TINY.layer_num):
            for a, b in zip(r.quant(name, layer), m.quant(name, layer)):
                np.testing.assert_array_equal(a, b)
    for a, b in zip(r.quant("cls"), m.quant("cls")):
        np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(r.fp32("embedding"), m.fp32("embedding"))
    for i in range(2 * TINY.layer_num + 1):
        np.testing.assert_array_equal(r.fp32("rmsnorm", i), m.fp32("rmsnorm", i))
    with pytest.raises(ValueError):
        mf.RandomModel(TINY_TIED, 64)


@pytest.mark.parametrize("cfg", [TINY, TINY_TIED])
def test_cpp_loader_offsets_match_layout(tmp_path, cfg):
    """The C++ loader (Int8ModelFile) binds every tensor at the offset the layout predicts."""
    path = mf.write_random(tmp_path / "m.bin", cfg, 64, seed=1)
    res = _cpp("dump", path)
    assert res.returncode == 0
    lines = res.stdout.splitlines()
    conf = next(ln for ln in lines if ln.startswith("config")).split()
    assert list(map(int, conf[1:12])) == [cfg.dim, cfg.hidden_dim, cfg.layer_num, cfg.head_num,
                                          cfg.kv_head_num, cfg.vocab, cfg.seq_len,
                                          int(cfg.shared), 64, cfg.kv_dim, cfg.dim // cfg.head_num]
    got = {}
    for ln in lines:
        p = ln.split()
        if p[0] == "quant":
            got[(p[1], int(p[2]))] = (int(p[3]), int(p[4]), int(p[5]), int(p[6]))
        elif p[0] == "fp32":
            got[(p[1], int(p[2]))] = int(p[3])
    for e in mf.layout(cfg, 64):
        if e.quantised:
            assert got[(e.name, e.layer)] == (e.rows, e.cols, e.offset, e.scale_offset), e
        else:
            assert got[(e.name, e.layer)] == e.offset, e
    end = int(next(ln for ln in lines if ln.startswith("end")).split()[1])
    assert end + 40 == mf.file_bytes(cfg, 64)


def test_cpp_loader_errors(tmp_path):
    """Missing file -> kPathNotValid (2); short file or bad header -> kModelParseError (3)."""
    path = mf.write_random(tmp_path / "m.bin", TINY, 64, seed=1)
    assert "status 0" in _cpp("status", path).stdout
    assert "status 2" in _cpp("status", tmp_path / "missing.bin").stdout
    raw = path.read_bytes()
    (tmp_path / "short.bin").write_bytes(raw[:-4])
    assert "status 3" in _cpp("status", tmp_path / "short.bin").stdout
    (tmp_path / "head.bin").write_bytes(raw[:20])
    assert "status 3" in _cpp("status", tmp_path / "head.bin").stdout
    bad = bytearray(raw)
    bad[36:40] = struct.pack("<i", 0)          # group size 0
    (tmp_path / "gs0.bin").write_bytes(bytes(bad))
    assert "status 3" in _cpp("status", tmp_path / "gs0.bin").stdout


@pytest.mark.gpu
def test_cpp_loader_forward_on_gpu(tmp_path):
    """Projections bound from a written file run on the GPU and match the oracle on the mapped
    bytes (M = 1, 2, 3, 8)."""
    cfg = mf.ModelConfig(dim=512, hidden_dim=1536, layer_num=2, head_num=8, kv_head_num=2,
                         vocab_size=-2000, seq_len=128)
    path = mf.write_random(tmp_path / "m.bin", cfg, 64, seed=5)
    res = _cpp("gpu", path, timeout=110)
    assert res.returncode == 0 and "gpu: 0 failure(s)" in res.stdout
