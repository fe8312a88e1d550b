"""Continuous batching on the GPU: the paged-KV operators of include/sq8_batch.h against the numpy
restatement (oracle/decode_oracle.py), and greedy-token identity of scheduled, chunked, preempted
batches (llm-steadyinfer_amd/scheduler.py + batch_model.py) with the float64 oracle decoding each
sequence alone."""
import importlib

import numpy as np
import pytest

from conftest import load_pkg
from oracle import decode_oracle as do

sq8_pkg = load_pkg()
mf = importlib.import_module("llm_steadyinfer_amd.model_file")

TINY = mf.ModelConfig(dim=256, hidden_dim=512, layer_num=2, head_num=4, kv_head_num=2,
                      vocab_size=-1000, seq_len=64, rope_theta=1e6)


def _t(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def test_batch_ops_reject_bad_arguments(sq8):
    L = sq8.lib()
    FAKE = 4096
    assert L.sq8_paged_rope_kv(None, 1, 4, 2, 64, FAKE, FAKE, 4, 16, FAKE, FAKE, FAKE, FAKE,
                               None) == sq8.SQ8_ERR_NULL
    assert L.sq8_paged_rope_kv(FAKE, 1, 4, 3, 64, FAKE, FAKE, 4, 16, FAKE, FAKE, FAKE, FAKE,
                               None) == sq8.SQ8_ERR_DIMS
    assert L.sq8_paged_attention(FAKE, 256, 1, 4, 2, 512, FAKE, FAKE, 4, 16, FAKE, FAKE, FAKE,
                                 None) == sq8.SQ8_ERR_DIMS
    assert L.sq8_paged_attention(FAKE, 100, 1, 4, 2, 64, FAKE, FAKE, 4, 16, FAKE, FAKE, FAKE,
                                 None) == sq8.SQ8_ERR_DIMS
    assert L.sq8_swiglu_rows(FAKE, 0, 8, FAKE, None) == sq8.SQ8_ERR_DIMS
    assert L.sq8_argmax_rows(None, 1, 8, FAKE, None) == sq8.SQ8_ERR_NULL


def _paged_case(rng, lens, kv, block_size, extra_blocks=7):
    """Contiguous per-sequence K/V and the same data scattered into shuffled physical blocks."""
    need = [(n + block_size - 1) // block_size for n in lens]
    nb = sum(need) + extra_blocks
    perm = rng.permutation(nb)
    kc = rng.standard_normal((nb, block_size, kv)).astype(np.float32)  # unowned blocks: noise
    vc = rng.standard_normal((nb, block_size, kv)).astype(np.float32)
    width = max(need) + 2
    tables, K, V, o = [], [], [], 0
    for n, b in zip(lens, need):
        blocks = perm[o:o + b]
        o += b
        tables.append(list(blocks) + [-1] * (width - b))
        k = rng.standard_normal((n, kv)).astype(np.float32)
        v = rng.standard_normal((n, kv)).astype(np.float32)
        for p in range(n):
            kc[blocks[p // block_size], p % block_size] = k[p]
            vc[blocks[p // block_size], p % block_size] = v[p]
        K.append(k)
        V.append(v)
    return kc, vc, tables, K, V


@pytest.mark.gpu
@pytest.mark.parametrize("heads,kv_heads,hs,block_size", [(4, 2, 64, 4), (12, 2, 128, 16),
                                                          (8, 8, 128, 32), (4, 1, 256, 16)])
def test_paged_attention_matches_oracle(sq8, dev, heads, kv_heads, hs, block_size):
    import torch
    rng = np.random.default_rng(heads * 100 + hs + block_size)
    lens = [1, 37, 200, 5, 64]
    kv = kv_heads * hs
    kc, vc, tables, K, V = _paged_case(rng, lens, kv, block_size)
    # rows: the last position of every sequence, plus several earlier positions of sequence 2
    rows = [(s, n - 1) for s, n in enumerate(lens)] + [(2, 0), (2, 17), (2, 150), (1, 36)]
    dim = heads * hs
    stride = dim + 2 * kv + 3  # q rows inside wider rows
    qkv = rng.standard_normal((len(rows), stride)).astype(np.float32)
    pos = np.array([p for _, p in rows], np.int32)
    tab = np.array([tables[s] for s, _ in rows], np.int32)
    out = torch.empty((len(rows), dim), device=dev)
    sq8.paged_attention(_t(qkv, dev), stride, heads, kv_heads, hs, _t(pos, dev), _t(tab, dev),
                        block_size, _t(kc, dev), _t(vc, dev), out)
    got = out.cpu().numpy()
    for i, (s, p) in enumerate(rows):
        ref = do.attention(qkv[i, :dim], K[s], V[s], p, heads, kv_heads, hs)
        err = np.max(np.abs(got[i] - ref)) / max(np.max(np.abs(ref)), 1e-30)
        assert err < 2e-6, (i, s, p, err)


def test_split_kv_workspace_bytes(sq8):
    """Split-KV workspace: none when a table row spans at most 128 positions, the row kernel does
    not cover the head shape or the table row does not fit its LDS; otherwise a ticket area of
    4096 rows x kv_head_num tickets (the same for every row count, so calls of different sizes
    on one workspace agree on where the partials start) plus G * (head_size + 2) floats per
    (work item, kv head), with
    768 / kv_head_num work items (fewer than 512 row-kv-head pairs) or rows, plus rows, at
    most over every row count up to rows."""
    f = sq8.paged_attention_workspace_bytes
    assert f(8, 32, 8, 128, 8, 16) == 0             # 128 positions: never split
    assert f(8, 32, 8, 256, 64, 16) == 0            # head_size 256: generic kernel
    assert f(8, 32, 8, 128, 4096, 16) == 0          # table row beyond the LDS stage
    assert f(8, 32, 8, 128, 16, 16) == 4096 * 8 * 4 + (96 + 8) * 8 * 4 * 130 * 4
    # 64 rows: 64 + 64 items; 63 rows (504 pairs): 96 + 63, the most for up to 64 rows
    assert f(64, 32, 8, 128, 68, 16) == 4096 * 8 * 4 + (96 + 63) * 8 * 4 * 130 * 4
    assert f(1, 28, 4, 64, 300, 4) == 4096 * 4 * 4 + (192 + 1) * 4 * 7 * 66 * 4
    assert f(3, 32, 8, 128, 68, 16) < f(4, 32, 8, 128, 68, 16)
    # total positions beyond 32 bits: 4096 rows never split, but calls of fewer rows may
    assert f(4096, 32, 8, 128, 4000, 256) >= f(2097, 32, 8, 128, 4000, 256) > 0


@pytest.mark.gpu
@pytest.mark.parametrize("heads,kv_heads,hs,block_size", [(32, 8, 128, 16), (4, 2, 64, 4),
                                                          (14, 2, 64, 1), (16, 2, 128, 32)])
def test_split_kv_attention_matches_oracle(sq8, dev, heads, kv_heads, hs, block_size):
    """Rows of 1..1500 positions cut into work items of at least 128 positions (chunk length set
    by the total over the rows) and merged by the last chunk to finish: equal to the oracle to
    the unsplit kernel's bound. Three calls on one workspace (9 rows, 64 rows at random
    positions, 3 rows) check that each call leaves its tickets ready for the next."""
    import torch
    rng = np.random.default_rng(heads + 7 * hs + block_size)
    lens = [1, 256, 257, 512, 1500, 700, 3]
    kv = kv_heads * hs
    kc, vc, tables, K, V = _paged_case(rng, lens, kv, block_size, extra_blocks=3)
    dim = heads * hs
    stride = dim + 2 * kv
    tab_all = np.array(tables, np.int32)
    many = [(s, int(rng.integers(0, lens[s]))) for s in rng.integers(0, len(lens), 64)]
    ws = torch.zeros((sq8.paged_attention_workspace_bytes(
        64, heads, kv_heads, hs, tab_all.shape[1], block_size) + 3) // 4,
        dtype=torch.int32, device=dev)
    assert ws.numel() > 0
    kc_t, vc_t = _t(kc, dev), _t(vc, dev)
    for rows in ([(s, n - 1) for s, n in enumerate(lens)] + [(4, 255), (4, 256)],
                 many, [(1, 255), (4, 1000), (5, 10)]):
        qkv = rng.standard_normal((len(rows), stride)).astype(np.float32)
        pos = np.array([p for _, p in rows], np.int32)
        tab = np.array([tables[s] for s, _ in rows], np.int32)
        out = torch.full((len(rows), dim), float("nan"), device=dev)
        sq8.paged_attention(_t(qkv, dev), stride, heads, kv_heads, hs, _t(pos, dev),
                            _t(tab, dev), block_size, kc_t, vc_t, out, workspace=ws)
        got = out.cpu().numpy()
        for i, (s, p) in enumerate(rows):
            ref = do.attention(qkv[i, :dim], K[s], V[s], p, heads, kv_heads, hs)
            err = np.max(np.abs(got[i] - ref)) / max(np.max(np.abs(ref)), 1e-30)
            assert err < 2e-6, (rows, i, s, p, err)
        assert int(ws[:4096 * kv_heads].abs().sum()) == 0  # tickets back at zero


@pytest.mark.gpu
def test_split_kv_small_call_then_large_call(sq8, dev):
    """One workspace shared by calls of different row counts: a 2-row call whose long row
    splits (its partials are written), then a 24-row call (24 x 8 kv heads > 64 tickets) whose
    rows split too, then the small call again. A partial area that moved with the call's row
    count would put the small call's partials on the large call's tickets; every output must
    match the oracle and the whole ticket area must be zero after each call."""
    import torch
    heads, kv_heads, hs, block_size = 32, 8, 128, 16
    rng = np.random.default_rng(2024)
    lens = [1200, 900, 700, 650, 30]
    kv = kv_heads * hs
    kc, vc, tables, K, V = _paged_case(rng, lens, kv, block_size, extra_blocks=3)
    dim = heads * hs
    stride = dim + 2 * kv
    width = len(tables[0])
    ws = torch.zeros((sq8.paged_attention_workspace_bytes(
        64, heads, kv_heads, hs, width, block_size) + 3) // 4, dtype=torch.int32, device=dev)
    kc_t, vc_t = _t(kc, dev), _t(vc, dev)
    small = [(0, 1199), (4, 29)]
    large = [(int(s), int(rng.integers(400, lens[s]))) for s in rng.integers(0, 4, 24)]
    for rows in (small, large, small, large):
        qkv = rng.standard_normal((len(rows), stride)).astype(np.float32)
        pos = np.array([p for _, p in rows], np.int32)
        tab = np.array([tables[s] for s, _ in rows], np.int32)
        out = torch.full((len(rows), dim), float("nan"), device=dev)
        sq8.paged_attention(_t(qkv, dev), stride, heads, kv_heads, hs, _t(pos, dev),
                            _t(tab, dev), block_size, kc_t, vc_t, out, workspace=ws)
        got = out.cpu().numpy()
        for i, (s, p) in enumerate(rows):
            ref = do.attention(qkv[i, :dim], K[s], V[s], p, heads, kv_heads, hs)
            err = np.max(np.abs(got[i] - ref)) / max(np.max(np.abs(ref)), 1e-30)
            assert err < 2e-6, (len(rows), i, s, p, err)
        assert int(ws[:4096 * kv_heads].abs().sum()) == 0


@pytest.mark.gpu
@pytest.mark.parametrize("heads,kv_heads,hs,block_size", [(4, 2, 64, 4), (12, 2, 128, 16)])
def test_paged_rope_kv_writes_slots(sq8, dev, heads, kv_heads, hs, block_size):
    import torch
    rng = np.random.default_rng(hs + block_size)
    max_seq, dim, kv = 256, heads * hs, kv_heads * hs
    width = max_seq // block_size          # a full table row per sequence, disjoint blocks
    nb = 3 * width + 5
    kc0 = np.full((nb, block_size, kv), -7.0, np.float32)
    tables = rng.permutation(nb)[:3 * width].reshape(3, width).astype(np.int32)
    rows = [(0, 0), (0, 1), (1, 77), (2, 255), (1, 5)]
    qkv = rng.standard_normal((len(rows), dim + 2 * kv)).astype(np.float32)
    sin = torch.empty((max_seq, hs), device=dev)
    cos = torch.empty((max_seq, hs), device=dev)
    sq8.rope_tables(sin, cos, hs, max_seq, 1e6)
    s_np, c_np = sin.cpu().numpy().astype(np.float64), cos.cpu().numpy().astype(np.float64)
    q_t, kc, vc = _t(qkv, dev), _t(kc0, dev), _t(kc0.copy(), dev)
    pos = np.array([p for _, p in rows], np.int32)
    tab = np.array([tables[s] for s, _ in rows], np.int32)
    sq8.paged_rope_kv(q_t, heads, kv_heads, hs, _t(pos, dev), _t(tab, dev), block_size, sin, cos,
                      kc, vc)
    q_out, k_out, v_out = q_t.cpu().numpy(), kc.cpu().numpy(), vc.cpu().numpy()
    written = set()
    for i, (s, p) in enumerate(rows):
        b, o = tables[s][p // block_size], p % block_size
        written.add((b, o))
        np.testing.assert_allclose(q_out[i, :dim], do.rope(qkv[i, :dim], heads, hs, p, s_np, c_np),
                                   rtol=0, atol=2e-6)
        np.testing.assert_allclose(k_out[b, o],
                                   do.rope(qkv[i, dim:dim + kv], kv_heads, hs, p, s_np, c_np),
                                   rtol=0, atol=2e-6)
        np.testing.assert_array_equal(v_out[b, o], qkv[i, dim + kv:])
    for b in range(nb):
        for o in range(block_size):
            if (b, o) not in written:
                assert np.all(k_out[b, o] == -7.0) and np.all(v_out[b, o] == -7.0)


@pytest.mark.gpu
def test_swiglu_and_argmax_rows(sq8, dev):
    import torch
    rng = np.random.default_rng(5)
    gu = (rng.standard_normal((7, 2 * 300)) * 3).astype(np.float32)
    out = torch.empty((7, 300), device=dev)
    sq8.swiglu_rows(_t(gu, dev), out)
    ref = do.swiglu(gu[:, :300], gu[:, 300:])
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=2e-6, atol=1e-6)
    lg = rng.standard_normal((6, 5003)).astype(np.float32)
    lg[1, 17] = lg[1, 4000] = 99.0            # tie: the first index wins
    lg[2, :] = -np.inf                        # all -inf: index 0
    lg[3, 10] = np.nan                        # NaN never wins
    lg[4, :] = np.nan                         # all NaN: 0
    idx = torch.empty(6, dtype=torch.int32, device=dev)
    sq8.argmax_rows(_t(lg, dev), idx)
    got = idx.cpu().numpy().tolist()
    assert got[1] == 17 and got[2] == 0 and got[4] == 0
    for r in (0, 3, 5):
        assert got[r] == int(np.nanargmax(lg[r]))


@pytest.mark.gpu
@pytest.mark.parametrize("max_batch,block_size,num_blocks,graphs,packed", [
    (4, 4, None, True, False), (4, 4, 20, True, False), (4, 4, 24, True, False),
    (8, 8, None, True, False), (96, 8, None, True, False), (8, 8, None, False, False)])
def test_continuous_batching_matches_oracle(sq8, dev, tmp_path, max_batch, block_size,
                                            num_blocks, graphs, packed):
    """Six prompts (1..40 tokens) scheduled with chunked prefill mixed into decode steps (and,
    with a 20- or 24-block pool, preemption and recompute): every sequence's greedy tokens equal the
    float64 oracle decoding it alone. Decode-only steps replay per-row-count HIP graphs between
    eager prefill steps (and run eagerly in the graphs=False case). With packed the model holds
    packed weights (sq8_pack_weights) and every matmul takes the _packed entry points."""
    sched = importlib.import_module("llm_steadyinfer_amd.scheduler")
    bm = importlib.import_module("llm_steadyinfer_amd.batch_model")
    dec = importlib.import_module("llm_steadyinfer_amd.decoder")
    path = mf.write_random(tmp_path / "m.bin", TINY, 64, seed=11, w_std=0.2)
    rng = np.random.default_rng(11)
    prompts = [rng.integers(0, TINY.vocab, n).tolist() for n in (5, 1, 23, 12, 40, 7)]
    n_new, max_seq = 12, 64
    ref = [do.DecodeModel(mf.ModelFile(path), max_seq=max_seq).generate(p, n_new)[0]
           for p in prompts]
    D = dec.Int8Decoder.from_file(path, max_seq=max_seq, device=dev)
    s = sched.Scheduler(None, max_batch=max_batch, max_seq_len=max_seq, max_gen_len=n_new,
                        block_size=block_size, num_blocks=num_blocks)
    model = bm.PagedBatchModel.from_decoder(D, max_rows=max_batch, max_seq_len=max_seq,
                                            num_blocks=s.alloc.num_blocks, block_size=block_size,
                                            use_graphs=graphs, packed=packed)
    s.forward = model.forward
    for p in prompts:
        assert s.add_request(p) >= 0
    done = s.run(max_steps=5000)
    got = [q.generated_tokens for q in done]
    print("steps", s.steps, "rows", s.rows_run, "preemptions", s.preemptions,
          "graph replays", model.graph_replays, "graphs", sorted(model.graphs))
    assert (model.graph_replays > 0) == graphs
    if num_blocks is not None:
        assert s.preemptions > 0
    if max_batch > 64:  # the 88 prompt tokens start as one step: the fused-epilogue GEMM path
        assert model.fused(88) == (True, True, True)
    if packed:
        assert all(isinstance(q, sq8.PackedWeight) for q, _ in model.w["qkv"])
    assert got == ref


@pytest.mark.gpu
def test_continuous_batching_long_rows_split_kv(dev, tmp_path):
    """Prompts of up to 300 tokens with a 320-position table row: attention rows past 256
    positions take the split-KV path (the model's workspace is allocated), in graph-replayed
    decode steps and eager prefill steps alike; every sequence's greedy tokens equal the float64
    oracle decoding it alone."""
    sched = importlib.import_module("llm_steadyinfer_amd.scheduler")
    bm = importlib.import_module("llm_steadyinfer_amd.batch_model")
    dec = importlib.import_module("llm_steadyinfer_amd.decoder")
    cfg = mf.ModelConfig(dim=256, hidden_dim=512, layer_num=2, head_num=4, kv_head_num=2,
                         vocab_size=-1000, seq_len=320, rope_theta=1e6)
    path = mf.write_random(tmp_path / "m.bin", cfg, 64, seed=12, w_std=0.2)
    rng = np.random.default_rng(12)
    prompts = [rng.integers(0, cfg.vocab, n).tolist() for n in (270, 5, 300, 256)]
    n_new, max_seq = 10, 320
    ref = [do.DecodeModel(mf.ModelFile(path), max_seq=max_seq).generate(p, n_new)[0]
           for p in prompts]
    D = dec.Int8Decoder.from_file(path, max_seq=max_seq, device=dev)
    s = sched.Scheduler(None, max_batch=4, max_seq_len=max_seq, max_gen_len=n_new, block_size=4)
    model = bm.PagedBatchModel.from_decoder(D, max_rows=4, max_seq_len=max_seq,
                                            num_blocks=s.alloc.num_blocks, block_size=4)
    assert model.att_ws is not None
    s.forward = model.forward
    for p in prompts:
        assert s.add_request(p) >= 0
    done = s.run(max_steps=5000)
    assert model.graph_replays > 0
    assert [q.generated_tokens for q in done] == ref


@pytest.mark.gpu
def test_prefix_cache_on_the_gpu_matches_oracle(dev, tmp_path):
    """Prefix cache with the HIP batch model: later requests mount the KV blocks of a running
    sequence that share their whole-block prompt prefix (block 8) and start their prefill after
    them; their greedy tokens equal the float64 oracle decoding each prompt alone. A stop token
    (the first request's 3rd token) retires sequences early."""
    sched = importlib.import_module("llm_steadyinfer_amd.scheduler")
    bm = importlib.import_module("llm_steadyinfer_amd.batch_model")
    dec = importlib.import_module("llm_steadyinfer_amd.decoder")
    path = mf.write_random(tmp_path / "m.bin", TINY, 64, seed=13, w_std=0.2)
    rng = np.random.default_rng(13)
    base = rng.integers(0, TINY.vocab, 24).tolist()
    first = base + [1, 2]
    later = [base + [3], base[:16] + [4, 5, 6], base[:8] + rng.integers(0, TINY.vocab, 9).tolist(),
             rng.integers(0, TINY.vocab, 10).tolist()]
    n_new, max_seq, bs = 12, 64, 8
    oracle = lambda p: do.DecodeModel(mf.ModelFile(path), max_seq=max_seq).generate(p, n_new)[0]
    ref = [oracle(p) for p in [first] + later]
    stop = ref[0][2]
    D = dec.Int8Decoder.from_file(path, max_seq=max_seq, device=dev)
    s = sched.Scheduler(None, max_batch=4, max_seq_len=max_seq, max_gen_len=n_new,
                        block_size=bs, prefix_cache=True, stop_tokens=[stop])
    model = bm.PagedBatchModel.from_decoder(D, max_rows=4, max_seq_len=max_seq,
                                            num_blocks=s.alloc.num_blocks, block_size=bs)
    s.forward = model.forward
    assert s.add_request(first) >= 0
    while not (s.running and s.running[0].prefill_complete):
        s.step()
    for p in later:
        assert s.add_request(p) >= 0
    done = s.run(max_steps=5000)
    print("shared blocks", s.shared_prefix_blocks, "steps", s.steps)
    assert s.shared_prefix_blocks >= 3 + 2 + 1
    for q, r in zip(done, ref):
        cut = next((k + 1 for k, t in enumerate(r) if t == stop), len(r))
        assert q.generated_tokens == r[:cut], q.id
    assert len(done[0].generated_tokens) == 3
