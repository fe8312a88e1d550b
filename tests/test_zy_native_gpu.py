"""GPU tests of the native (C++) host side: scheduler::Scheduler driving the HIP batch model,
model::PagedBatchModel, model::Int8Decoder and the all-C++ path from a model file
(model::DeviceWeights). Each compares greedy tokens with the float64 oracle and with the Python
host side, which issues the same libsq8 calls (checked on the CPU by
tests/test_native_scheduler.py). Collected after the kernel parity tests."""
import importlib

import numpy as np
import pytest

from conftest import load_pkg
from oracle import decode_oracle as do

sq8 = load_pkg()
mf = importlib.import_module("llm_steadyinfer_amd.model_file")
TINY = mf.ModelConfig(dim=256, hidden_dim=512, layer_num=2, head_num=4, kv_head_num=2,
                      vocab_size=-1000, seq_len=64, rope_theta=1e6)
TINY_MHA = mf.ModelConfig(dim=256, hidden_dim=640, layer_num=3, head_num=2, kv_head_num=2,
                          vocab_size=-777, seq_len=64, rope_theta=5e5)


def _decoder_mod():
    return importlib.import_module("llm_steadyinfer_amd.decoder")


@pytest.mark.gpu
def test_native_scheduler_drives_the_batch_model(dev, tmp_path):
    """The native scheduler (scheduler::Scheduler through native_scheduler.py) drives the HIP
    batch model over its array entry point, with preemption and decode graphs; every sequence's
    greedy tokens equal the float64 oracle decoding it alone."""
    nat = importlib.import_module("llm_steadyinfer_amd.native_scheduler")
    bm = importlib.import_module("llm_steadyinfer_amd.batch_model")
    dec = importlib.import_module("llm_steadyinfer_amd.decoder")
    path = mf.write_random(tmp_path / "m.bin", TINY, 64, seed=14, w_std=0.2)
    rng = np.random.default_rng(14)
    prompts = [rng.integers(0, TINY.vocab, n).tolist() for n in (5, 1, 23, 12, 40, 7)]
    n_new, max_seq, bs, nblocks = 12, 64, 4, 24
    ref = [do.DecodeModel(mf.ModelFile(path), max_seq=max_seq).generate(p, n_new)[0]
           for p in prompts]
    D = dec.Int8Decoder.from_file(path, max_seq=max_seq, device=dev)
    model = bm.PagedBatchModel.from_decoder(D, max_rows=4, max_seq_len=max_seq,
                                            num_blocks=nblocks, block_size=bs)
    s = nat.NativeScheduler(model, max_batch=4, max_seq_len=max_seq, max_gen_len=n_new,
                            block_size=bs, num_blocks=nblocks)
    for p in prompts:
        assert s.add_request(p) >= 0
    done = s.run(max_steps=5000)
    print("steps", s.steps, "rows", s.rows_run, "preemptions", s.preemptions,
          "graph replays", model.graph_replays)
    assert s.preemptions > 0 and model.graph_replays > 0
    assert [q.generated_tokens for q in done] == ref


@pytest.mark.gpu
@pytest.mark.parametrize("packed", [False, True])
def test_native_model_and_scheduler_match_oracle(dev, tmp_path, packed):
    """model::PagedBatchModel (C++) driven by scheduler::Scheduler (C++) with no Python in the
    step loop: preemption, decode graphs and split-KV rows (prompts past 128 positions); every
    sequence's greedy tokens equal the float64 oracle, and the Python model under the Python
    scheduler gives the same tokens."""
    nat = importlib.import_module("llm_steadyinfer_amd.native_scheduler")
    sched = importlib.import_module("llm_steadyinfer_amd.scheduler")
    bm = importlib.import_module("llm_steadyinfer_amd.batch_model")
    dec = importlib.import_module("llm_steadyinfer_amd.decoder")
    cfg = mf.ModelConfig(dim=256, hidden_dim=512, layer_num=2, head_num=4, kv_head_num=2,
                         vocab_size=-1000, seq_len=320, rope_theta=1e6)
    path = mf.write_random(tmp_path / "m.bin", cfg, 64, seed=15, w_std=0.2)
    rng = np.random.default_rng(15)
    prompts = [rng.integers(0, cfg.vocab, n).tolist() for n in (270, 5, 33, 140, 1, 12)]
    n_new, max_seq, bs, nblocks = 10, 320, 4, 90
    ref = [do.DecodeModel(mf.ModelFile(path), max_seq=max_seq).generate(p, n_new)[0]
           for p in prompts]
    D = dec.Int8Decoder.from_file(path, max_seq=max_seq, device=dev)
    model = nat.NativePagedBatchModel(D.cfg, D.w, D.gs, max_rows=4, max_seq_len=max_seq,
                                      num_blocks=nblocks, block_size=bs, packed=packed)
    print("native model created", flush=True)
    model.capture_decode_graphs()
    s = nat.NativeScheduler(model, max_batch=4, max_seq_len=max_seq, max_gen_len=n_new,
                            block_size=bs, num_blocks=nblocks)
    for p in prompts:
        assert s.add_request(p) >= 0
    done = s.run(max_steps=5000)
    print("steps", s.steps, "preemptions", s.preemptions, "graph replays", model.graph_replays,
          flush=True)
    assert s.preemptions > 0 and model.graph_replays > 0
    got = [q.generated_tokens for q in done]
    assert got == ref
    s2 = sched.Scheduler(None, max_batch=4, max_seq_len=max_seq, max_gen_len=n_new,
                         block_size=bs, num_blocks=nblocks)
    pm = bm.PagedBatchModel.from_decoder(D, max_rows=4, max_seq_len=max_seq, num_blocks=nblocks,
                                         block_size=bs, packed=packed)
    s2.forward = pm.forward
    for p in prompts:
        s2.add_request(p)
    assert [q.generated_tokens for q in s2.run(max_steps=5000)] == got


@pytest.mark.gpu
def test_native_batch_model_from_file_matches_oracle(dev, tmp_path):
    """The all-C++ continuous-batching path: model file -> model::DeviceWeights ->
    model::PagedBatchModel driven by scheduler::Scheduler; tokens equal the oracle's."""
    nat = importlib.import_module("llm_steadyinfer_amd.native_scheduler")
    path = mf.write_random(tmp_path / "m.bin", TINY, 64, seed=23, w_std=0.2)
    rng = np.random.default_rng(23)
    prompts = [rng.integers(0, TINY.vocab, n).tolist() for n in (9, 1, 30, 17)]
    n_new, max_seq, bs = 10, 64, 8
    ref = [do.DecodeModel(mf.ModelFile(path), max_seq=max_seq).generate(p, n_new)[0]
           for p in prompts]
    model = nat.NativePagedBatchModel.from_file(path, max_rows=4, max_seq_len=max_seq,
                                                num_blocks=4 * (max_seq // bs), block_size=bs)
    print("native batch model from file created", flush=True)
    s = nat.NativeScheduler(model, max_batch=4, max_seq_len=max_seq, max_gen_len=n_new,
                            block_size=bs)
    for p in prompts:
        assert s.add_request(p) >= 0
    assert [q.generated_tokens for q in s.run(max_steps=5000)] == ref


@pytest.mark.gpu
@pytest.mark.parametrize("use_graph", [True, False])
def test_native_decoder_matches_python_decoder_and_oracle(dev, tmp_path, use_graph):
    """model::Int8Decoder (C++ host loop, one graph replay per token) on the weights of the
    Python decoder: greedy tokens equal the Python decoder's and the float64 oracle's."""
    nat = importlib.import_module("llm_steadyinfer_amd.native_scheduler")
    cfg = mf.ModelConfig(dim=256, hidden_dim=512, layer_num=2, head_num=4, kv_head_num=2,
                         vocab_size=-1000, seq_len=96, rope_theta=1e6)
    path = mf.write_random(tmp_path / "m.bin", cfg, 64, seed=21, w_std=0.2)
    prompt = np.random.default_rng(21).integers(0, cfg.vocab, 17).tolist()
    D = _decoder_mod().Int8Decoder.from_file(path, max_seq=96, device=dev)
    ref = do.DecodeModel(mf.ModelFile(path), max_seq=96).generate(prompt, 12)[0]
    N = nat.NativeInt8Decoder(D.cfg, D.w, D.gs, max_seq=96)
    print("native decoder created", flush=True)
    got = N.generate(prompt, 12, use_graph=use_graph)
    assert got == ref
    assert N.generate(prompt, 12, use_graph=use_graph) == got  # reset between runs
    assert D.generate(prompt, 12) == got


@pytest.mark.gpu
def test_native_decoder_from_file_matches_oracle(dev, tmp_path):
    """The all-C++ path: the INT8 model file read by model::Int8ModelFile, uploaded fused by
    model::DeviceWeights, decoded by model::Int8Decoder; greedy tokens equal the oracle's."""
    nat = importlib.import_module("llm_steadyinfer_amd.native_scheduler")
    path = mf.write_random(tmp_path / "m.bin", TINY_MHA, 64, seed=22, w_std=0.2)
    prompt = np.random.default_rng(22).integers(0, TINY_MHA.vocab, 9).tolist()
    ref = do.DecodeModel(mf.ModelFile(path), max_seq=64).generate(prompt, 16)[0]
    N = nat.NativeInt8Decoder.from_file(path, max_seq=64)
    print("native decoder from file created", flush=True)
    assert N.generate(prompt, 16) == ref
