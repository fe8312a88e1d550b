"""Greedy-token identity at the real widths of the end-to-end configurations.

Config 5 (continuous batching): 64 requests with lognormal prompt lengths (median 200, sigma 0.8,
clipped 16..2048: the bench's own draw), 128 greedy tokens each, paged KV block 16, max_batch 64,
through Scheduler + PagedBatchModel, on a model with Llama-3-8B layer geometry (dim 4096, 32 / 8
heads, head 128, FFN 14336, group 64, rope theta 5e5) cut to 2 layers and a 16384-token vocab.
- 4 sequences (the shortest, the longest and two in between): the first 8 tokens equal the
  float64 oracle decoding the sequence alone (oracle/decode_oracle.py).
- All 64: the 128 tokens equal the HIP single-sequence decoder (Int8Decoder, contiguous KV, M=1
  GEMV path) decoding the sequence alone: batch invariance across the 1..64-row kernels, chunked
  prefill, split-KV attention and the decode-graph pool.

Config 4 (single-sequence decode): a Qwen2-1.5B-width model (dim 1536, 12 / 2 heads, FFN 8960,
the full 151936-token vocab) cut to 4 layers, a 64-token prompt and 24 greedy tokens on the
HIP-graph decoder against the float64 oracle.

Near ties. The oracle sums in float64 and the kernels in fp32, so the two can only disagree where
the top two logits are closer than fp32 rounding of the sum (about 1e-6 of the logit scale). A
disagreement is accepted only at such a near tie: the reference side's top-2 gap must be below
NEAR_TIE x its largest |logit|, the kernel's token must be the runner-up, and the sequence is
compared no further (its contexts differ from there on). Every such event is printed; the test
fails on any other disagreement and on more than MAX_TIES of them.

The reference's own verification is the same kind of A/B: greedy tokens of its paged batched run
against its contiguous single-sequence run (benchmark/verify_tokens.cpp:1-74).
"""
import importlib

import numpy as np
import pytest

from conftest import load_pkg
from oracle import decode_oracle as do

load_pkg()
mf = importlib.import_module("llm_steadyinfer_amd.model_file")

NEAR_TIE = 1e-5
MAX_TIES = 2

LLAMA_2L = mf.ModelConfig(dim=4096, hidden_dim=14336, layer_num=2, head_num=32, kv_head_num=8,
                          vocab_size=-16384, seq_len=8192, rope_theta=500000.0)
QWEN_4L = mf.ModelConfig(dim=1536, hidden_dim=8960, layer_num=4, head_num=12, kv_head_num=2,
                         vocab_size=-151936, seq_len=8192, rope_theta=1000000.0)


def config5_prompts(vocab: int, n_seqs: int = 64, seed: int = 0, sigma: float = 0.8):
    """bench.py's config-5 draw: lognormal lengths (median 200) clipped to 16..2048, uniform ids."""
    rng = np.random.default_rng(seed)
    lens = np.clip(np.rint(np.exp(rng.normal(np.log(200.0), sigma, n_seqs))), 16, 2048)
    return [rng.integers(0, vocab, int(n)).tolist() for n in lens]


def top2_gap(logits):
    lg = np.asarray(logits, np.float64)
    i = int(np.argmax(lg))
    rest = np.delete(lg, i)
    j = int(np.argmax(rest))
    return lg[i] - rest[j], (j if j < i else j + 1), float(np.max(np.abs(lg)))


def compare(name, got, want, logits_at, ties):
    """Token lists equal, or equal up to a near tie at the first difference (see module doc)."""
    for i, (g, w) in enumerate(zip(got, want)):
        if g == w:
            continue
        gap, second, scale = top2_gap(logits_at(i))
        print(f"{name}: token {i} differs ({g} vs {w}); reference top-2 gap {gap:.3e}, "
              f"scale {scale:.3e}, runner-up {second}")
        assert gap < NEAR_TIE * scale and g == second, f"{name}: not a near tie at token {i}"
        ties.append((name, i))
        return
    assert len(got) == len(want), name


@pytest.mark.gpu
@pytest.mark.timeout(900)
def test_config5_llama_geometry_batch_matches_oracle_and_single_decoder(dev):
    import torch
    sched = importlib.import_module("llm_steadyinfer_amd.scheduler")
    bm = importlib.import_module("llm_steadyinfer_amd.batch_model")
    dec = importlib.import_module("llm_steadyinfer_amd.decoder")
    cfg, n_new = LLAMA_2L, 128
    m = mf.RandomModel(cfg, 64, seed=5)
    prompts = config5_prompts(cfg.vocab)
    lens = [len(p) for p in prompts]
    max_seq = max(lens) + n_new
    print(f"config 5 geometry: {len(prompts)} prompts, mean {np.mean(lens):.0f}, "
          f"max {max(lens)}, total {sum(lens)}", flush=True)
    D = dec.Int8Decoder.from_model(m, max_seq=max_seq, device=dev)
    block = sched.Scheduler.resolve_block_size(float(np.mean(lens)))
    assert block == 16
    s = sched.Scheduler(None, max_batch=64, max_seq_len=max_seq, max_gen_len=n_new,
                        block_size=block)
    model = bm.PagedBatchModel.from_decoder(D, max_rows=64, max_seq_len=max_seq,
                                            num_blocks=s.alloc.num_blocks, block_size=block)
    model.capture_decode_graphs()
    s.forward = model.forward
    for p in prompts:
        assert s.add_request(p) >= 0
    done = s.run(max_steps=20000)
    batch = [q.generated_tokens for q in done]
    print(f"scheduled: {s.steps} steps, {s.rows_run} rows, {s.preemptions} preemptions, "
          f"{model.graph_replays} graph replays", flush=True)
    assert model.graph_replays > 0 and model.att_ws is not None
    assert all(len(t) == n_new for t in batch)
    # The row counts the run used cover the tile, decode-GEMM and prefill-GEMM kernels.
    assert max(lens) > 256  # split-KV rows

    ties = []
    # Batch invariance: every sequence alone on the single-sequence HIP decoder.
    single = []
    for i, p in enumerate(prompts):
        single.append(D.generate(p, n_new))

    def single_logits(i):
        def at(t):
            D.generate(prompts[i], t + 1, use_graph=False)
            torch.cuda.synchronize()
            return D.logits.cpu().numpy()
        return at

    for i in range(len(prompts)):
        compare(f"seq {i} batch vs single", batch[i], single[i], single_logits(i), ties)

    # Oracle identity on four sequences (first 8 tokens).
    order = np.argsort(lens)
    pick = sorted({int(order[0]), int(order[-1]), int(order[len(order) // 3]),
                   int(order[2 * len(order) // 3])})
    oracle = do.DecodeModel(m, max_seq=max_seq)  # generate() overwrites the cache rows it reads
    for i in pick:
        ref, logits = oracle.generate(prompts[i], 8, batched_prompt=True)
        gaps = [top2_gap(lg)[0] for lg in logits]
        print(f"seq {i} (prompt {lens[i]}): oracle {ref}, smallest top-2 gap {min(gaps):.3e}",
              flush=True)
        compare(f"seq {i} batch vs oracle", batch[i][:8], ref, lambda t: logits[t], ties)
        compare(f"seq {i} single vs oracle", single[i][:8], ref, lambda t: logits[t], ties)
    print("near ties:", ties)
    assert len(ties) <= MAX_TIES


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_config4_qwen2_width_decoder_matches_oracle(dev):
    dec = importlib.import_module("llm_steadyinfer_amd.decoder")
    cfg, n_new = QWEN_4L, 24
    m = mf.RandomModel(cfg, 64, seed=4)
    prompt = np.random.default_rng(4).integers(0, cfg.vocab, 64).tolist()
    D = dec.Int8Decoder.from_model(m, max_seq=128, device=dev)
    got = D.generate(prompt, n_new)                 # HIP graph per token
    eager = D.generate(prompt, n_new, use_graph=False)
    assert got == eager
    ref, logits = do.DecodeModel(m, max_seq=128).generate(prompt, n_new, batched_prompt=True)
    gaps = [top2_gap(lg)[0] for lg in logits]
    print(f"oracle {ref}\nsmallest top-2 gap {min(gaps):.3e}, logit scale "
          f"{float(np.max(np.abs(logits[0]))):.3e}")
    ties = []
    compare("config 4", got, ref, lambda t: logits[t], ties)
    assert not ties or len(got) == n_new
    assert len(ties) <= 1
