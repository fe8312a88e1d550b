#!/usr/bin/env python3
"""Benchmark of the gfx950 INT8 group-quant matmul path on one MI355X.

A "step" is the INT8 matmul work of one Llama-3-8B decode token at batch 1 (the batched-decode
configuration at M=1): for each of the 32 layers the fused QKV (6144x4096), O (4096x4096), fused gate/up
(28672x4096) and down (4096x14336) projections, then the LM head (128256x4096). All 129 weights
are distinct random-init INT8 tensors resident in HBM (7.97 GB with scales), so no launch finds its
weight in the 256 MB Infinity Cache. `value` is algorithmic bytes per step / step time (GB/s).

Also reported: the per-launch GB/s and TFLOP/s of every (projection, M) pair of the batched-decode
(M in 1, 8, 32, 64) and prefill (M = 2048) configurations,
the roofline of the dominant kernel, and the CPU oracle's throughput on a bounded sample.
Counter runs: `python bench.py --profile` (see profiles/ for the rocprofv3 commands).

The step's 129 launches are issued eagerly on one stream; `--graph` replays them as one HIP graph
instead (the reference captures its decode step in a CUDA graph, src/source/model/model.cpp:
189-238). On MI355X the eager launches measured faster, so eager is the default.

Decode tokens/s (the metric's second half) comes from config 4: a Qwen2-1.5B-shaped random-init
INT8 model (28 layers, hidden 1536, 12 Q / 2 KV heads, FFN 8960, vocab 151936) decoding 128
greedy tokens at batch 1 after a 64-token prompt, on the HIP decode stack (decoder.py), each token
one HIP-graph replay; `--no-decode` skips it.

Config 5 (continuous batching): 64 requests with lognormal prompt lengths (median 200) on the
Llama-3-8B-shaped model (the step's weights plus a random embedding), 128 greedy tokens each,
through the paged-KV scheduler (scheduler.py) and batched model (batch_model.py): output
tokens/s over the wall time of the whole run; `--no-batch` skips it.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-sweep] [--no-cpu] [--no-decode]
                       [--no-batch] [--graph]
       python bench.py --profile   # short run for rocprofv3 counter passes (see profiles/)
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
GS = 64
HIDDEN, FFN, VOCAB, LAYERS = 4096, 14336, 128256, 32
PROJ = {"qkv": (6144, HIDDEN), "o": (HIDDEN, HIDDEN), "gate_up": (2 * FFN, HIDDEN),
        "down": (HIDDEN, FFN)}
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense f16 matrix peak (the prefill GEMM issues f16 MFMA)
# HBM bytes per M=1 GEMV launch over algorithmic bytes, from rocprofv3 FETCH_SIZE/WRITE_SIZE passes
# over `python bench.py --profile`, scaled by a 256 MiB copy of known size (profiles/).
GEMV_TRAFFIC_RATIO = 1.004
METRIC = "INT8 GEMV HBM GB/s (% of peak) + decode tokens/s, Llama-3-8B shapes, 1 GPU"


def load_pkg():
    name = "llm_steadyinfer_amd"
    pkg_dir = REPO / "llm-steadyinfer_amd"
    spec = importlib.util.spec_from_file_location(name, pkg_dir / "__init__.py",
                                                  submodule_search_locations=[str(pkg_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def algo_bytes(M, N, K, gs=GS):
    """Each operand byte counted once: int8 W, fp32 scales, fp32 x, fp32 y."""
    return N * K + 4 * (N * K // gs) + 4 * M * K + 4 * M * N


def make_q8(torch, N, K, gen, dev):
    """Random-init INT8 weight: W ~ N(0, 0.02) quantised per 64-group with absmax/127 scales."""
    q = torch.empty((N, K), dtype=torch.int8, device=dev)
    s = torch.empty((N * K // GS,), dtype=torch.float32, device=dev)
    rows = max(1, (1 << 26) // K)
    for r0 in range(0, N, rows):
        r1 = min(N, r0 + rows)
        w = torch.randn((r1 - r0, K), generator=gen, device=dev, dtype=torch.float32) * 0.02
        g = w.view(r1 - r0, K // GS, GS)
        sc = g.abs().amax(-1) / 127.0
        v = g / torch.where(sc == 0, torch.ones_like(sc), sc).unsqueeze(-1)
        qq = torch.sign(v) * torch.floor(v.abs() + 0.5)
        q[r0:r1] = qq.clamp_(-127, 127).to(torch.int8).view(r1 - r0, K)
        s[r0 * K // GS:r1 * K // GS] = sc.reshape(-1)
    return q, s


class Call:
    """Pre-bound sq8_matmul call (raw pointers) so the host loop adds little per launch."""

    def __init__(self, sq8, x, q, s, y, stream, ws):
        M, K = x.shape
        N = q.shape[0]
        packed = isinstance(q, sq8.PackedWeight)
        self.fn = sq8.lib().sq8_matmul_packed if packed else sq8.lib().sq8_matmul
        wsb = (int(sq8.lib().sq8_packed_workspace_bytes(M, N, K, GS)) if packed
               else sq8.workspace_bytes(M, N, K, GS))
        ws_ptr, ws_n = ws.get(wsb)
        self.args = (x.data_ptr(), q.data_ptr(), s.data_ptr(), y.data_ptr(), M, N, K, GS,
                     ws_ptr or None, ws_n, stream.cuda_stream)
        self.M, self.N, self.K = M, N, K
        self.bytes = algo_bytes(M, N, K)
        self.flops = 2 * M * N * K

    def __call__(self):
        rc = self.fn(*self.args)
        if rc != 0:
            raise RuntimeError(f"sq8 matmul failed with status {rc}")


def cpu_baseline(torch, weights, budget_s=10.0):
    """Oracle CPU loop (reference CPU GEMM structure, OpenMP) on one layer's four projections at
    M=1: one rep = the four calls; reps repeated for about budget_s seconds (at least 10). Returns
    the median rep's GB/s by the same byte formula, with the spread."""
    sys.path.insert(0, str(REPO))
    import numpy as np
    from oracle import sq8_oracle as o
    layer = [(p, weights[p][0][0].cpu().numpy(), weights[p][0][1].cpu().numpy()) for p in PROJ]
    rng = np.random.default_rng(0)
    xs = {p: rng.standard_normal((1, PROJ[p][1]), dtype=np.float32) for p in PROJ}
    for p, q, s in layer:  # warm-up
        o.matmul_cpu_loop(xs[p], q, s, GS)
    rep_bytes = sum(algo_bytes(1, *PROJ[p]) for p in PROJ)
    times, t0 = [], time.perf_counter()
    while len(times) < 10 or time.perf_counter() - t0 < budget_s:
        a = time.perf_counter()
        for p, q, s in layer:
            o.matmul_cpu_loop(xs[p], q, s, GS)
        times.append(time.perf_counter() - a)
    rates = sorted(rep_bytes / t / 1e9 for t in times)
    med = float(np.median(rates))
    # The batched-decode rows too: the same loop at M = 8 and 64 on the same layer, a bounded
    # sample each (median of at least 3 reps, about budget_s / 4 seconds).
    sweep = []
    for M in (8, 64):
        xm = {p: rng.standard_normal((M, PROJ[p][1]), dtype=np.float32) for p in PROJ}
        mb = sum(algo_bytes(M, *PROJ[p]) for p in PROJ)
        mf = sum(2.0 * M * PROJ[p][0] * PROJ[p][1] for p in PROJ)
        ts, t1 = [], time.perf_counter()
        while len(ts) < 3 or time.perf_counter() - t1 < budget_s / 4:
            a = time.perf_counter()
            for p, q, s in layer:
                o.matmul_cpu_loop(xm[p], q, s, GS)
            ts.append(time.perf_counter() - a)
        tm = float(np.median(ts))
        sweep.append({"M": M, "GB/s": round(mb / tm / 1e9, 2), "GFLOP/s": round(mf / tm / 1e9, 1),
                      "reps": len(ts)})
    return {"value": round(med, 2), "unit": "GB/s", "cores": o.max_threads(), "kind": "port",
            "sweep": sweep,
            "statistic": f"median of {len(times)} reps (min {rates[0]:.1f}, max {rates[-1]:.1f})",
            "sample": "oracle sq8o_matmul_cpu_loop (reference CPU GEMM loop, OpenMP), M=1, one "
                      "rep = one Llama-3-8B layer's qkv, o, gate_up and down projections, "
                      f"{time.perf_counter() - t0:.1f} s"}


def decode_run(torch, n_prompt: int = 64, n_new: int = 128, seed: int = 0):
    """Config 4: greedy decode on a Qwen2-1.5B-shaped random-init INT8 model (on-device init of the
    model-file distribution). The prompt runs eagerly one token per step (not timed as decode);
    the n_new decode tokens are graph replays timed with HIP events on the current stream."""
    import importlib
    import numpy as np
    mf = importlib.import_module("llm_steadyinfer_amd.model_file")
    dec = importlib.import_module("llm_steadyinfer_amd.decoder")
    cfg = mf.QWEN2_1_5B
    D = dec.Int8Decoder.random(cfg, max_seq=n_prompt + n_new, seed=seed)
    prompt = np.random.default_rng(seed).integers(0, cfg.vocab, n_prompt).tolist()
    D.generate(prompt, 4)                      # captures the graph, warms every kernel
    st = torch.cuda.current_stream()
    D.reset()
    t0 = time.perf_counter()
    for t in prompt[:-1]:
        D.token.fill_(int(t))
        D._launch_step(st, want_logits=False)
    D.token.fill_(int(prompt[-1]))
    D.begin_decode(st)
    torch.cuda.synchronize()
    prompt_ms = (time.perf_counter() - t0) * 1e3
    toks = torch.empty(n_new, dtype=torch.int32, device=D.device)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    for i in range(n_new):
        D.graph.replay()
        toks[i:i + 1].copy_(D.token)
    b.record(st)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / n_new
    wb = D.weight_bytes()
    return {"workload": "config 4: Qwen2-1.5B-shaped random-init INT8 model (28 layers, hidden "
                        "1536, 12/2 heads, FFN 8960, vocab 151936, group 64), batch 1, "
                        f"{n_prompt}-token prompt, {n_new} greedy tokens",
            "tokens_per_s": round(1e3 / ms, 1), "ms_per_token": round(ms, 4),
            "prompt_ms_eager": round(prompt_ms, 1), "weight_bytes_per_token": wb,
            "weight_GBps": round(wb / ms / 1e6, 1), "launch": "hip_graph per token",
            "first_tokens": toks[:8].cpu().tolist()}


def llama_decode_run(torch, weights, lm_head, n_prompt: int = 64, n_new: int = 128,
                     seed: int = 0):
    """Batch-1 greedy decode on the Llama-3-8B-shaped INT8 model (the step's random-init
    projections, a random embedding, unit norms) through the HIP decode stack (decoder.py: the
    reference's single-token LLamaModel::predict / forward, llama3.cpp:705-818), one HIP-graph
    replay per token, timed with HIP events; the 64-token prompt runs eagerly, untimed."""
    import importlib
    import numpy as np
    mf = importlib.import_module("llm_steadyinfer_amd.model_file")
    dec = importlib.import_module("llm_steadyinfer_amd.decoder")
    cfg = mf.LLAMA3_8B
    dev = lm_head[0].device
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed + 99)
    w = {"qkv": weights["qkv"], "o": weights["o"], "gu": weights["gate_up"],
         "down": weights["down"], "cls": lm_head,
         "emb": torch.randn((cfg.vocab, cfg.dim), generator=gen, device=dev),
         "norm": [torch.ones(cfg.dim, device=dev) for _ in range(2 * cfg.layer_num + 1)]}
    D = dec.Int8Decoder(cfg, w, GS, n_prompt + n_new, device=dev)
    prompt = np.random.default_rng(seed).integers(0, cfg.vocab, n_prompt).tolist()
    D.generate(prompt, 4)                      # captures the graph, warms every kernel
    st = torch.cuda.current_stream()
    D.reset()
    for t in prompt[:-1]:
        D.token.fill_(int(t))
        D._launch_step(st, want_logits=False)
    D.token.fill_(int(prompt[-1]))
    D.begin_decode(st)
    toks = torch.empty(n_new, dtype=torch.int32, device=dev)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    for i in range(n_new):
        D.graph.replay()
        toks[i:i + 1].copy_(D.token)
    b.record(st)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / n_new
    wb = D.weight_bytes()
    return {"workload": "Llama-3-8B-shaped random-init INT8 model (32 layers, hidden 4096, 32/8 "
                        "heads, FFN 14336, vocab 128256, group 64), batch 1, "
                        f"{n_prompt}-token prompt, {n_new} greedy tokens",
            "tokens_per_s": round(1e3 / ms, 1), "ms_per_token": round(ms, 4),
            "weight_bytes_per_token": wb, "weight_GBps": round(wb / ms / 1e6, 1),
            "frac_of_hbm_peak": round(wb / ms / 1e6 / HBM_PEAK_GBS, 4),
            "launch": "hip_graph per token", "first_tokens": toks[:8].cpu().tolist()}


def read_ceiling(torch, sq8, dev, shapes):
    """The read-only streaming probe (include/sq8_probe.h) over as many bytes as each shape's M=1
    GEMV reads, back to back over buffers rotated through > 1 GB, at a few grid and load-depth
    settings; the fastest setting is the ceiling a kernel reading those bytes once can reach."""
    out = {}
    sink = torch.zeros(4096, dtype=torch.int32, device=dev)
    for name, nbytes in shapes:
        n = (nbytes + 255) // 256 * 256
        nbuf = max(2, min(16, (1 << 30) // n + 1))
        bufs = [torch.empty(n, dtype=torch.uint8, device=dev) for _ in range(nbuf)]
        best = None
        fn = sq8.lib().sq8_probe_stream_read
        st = torch.cuda.current_stream().cuda_stream
        for wpc, u in ((4, 4), (8, 4), (8, 2), (16, 2), (4, 8), (2, 8), (16, 4), (32, 1)):
            args = [(b.data_ptr(), n, sink.data_ptr(), sink.numel(), wpc, u, st) for b in bufs]
            for a_ in args:
                fn(*a_)
            reps = 4 * nbuf
            a, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for i in range(reps):
                fn(*args[i % nbuf])
            e.record()
            torch.cuda.synchronize()
            us = a.elapsed_time(e) * 1e3 / reps
            if best is None or us < best[0]:
                best = (us, wpc, u)
        out[name] = {"bytes": n, "us": round(best[0], 2), "GB/s": round(n / best[0] / 1e3, 1),
                     "workgroups_per_cu": best[1], "chunks_per_lane": best[2]}
        del bufs
    return out


def copy_ceiling(torch, dev, shapes):
    """Device-to-device copies moving as many HBM bytes (read + write) as each shape's M=1 GEMV
    reads, back to back over buffers rotated through > 1 GB (so the 256 MB Infinity Cache cannot
    serve them): the box's streaming ceiling at that transfer size, launch floor included."""
    out = {}
    for name, nbytes in shapes:
        half = (nbytes // 2 + 255) // 256 * 256
        nbuf = max(2, min(16, (1 << 30) // half + 1))
        src = [torch.empty(half, dtype=torch.uint8, device=dev) for _ in range(nbuf)]
        dst = [torch.empty(half, dtype=torch.uint8, device=dev) for _ in range(nbuf)]
        for i in range(nbuf):
            dst[i].copy_(src[i])
        reps = 4 * nbuf
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for i in range(reps):
            dst[i % nbuf].copy_(src[i % nbuf])
        b.record()
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / reps
        out[name] = {"bytes_moved": 2 * half, "us": round(us, 2),
                     "GB/s": round(2 * half / us / 1e3, 1)}
        del src, dst
    return out


def batch_run(torch, weights, lm_head, n_seqs: int = 64, n_new: int = 128, seed: int = 0,
              sigma: float = 0.8, packed: bool = False, native: bool = False,
              native_model: bool = False):
    """Config 5: continuous batching of n_seqs requests on the Llama-3-8B-shaped INT8 model (the
    step's random-init projections, plus a random embedding and unit norms). Prompt lengths are
    lognormal with median 200 (sigma 0.8, clipped to 16..2048), uniform random token ids,
    n_new greedy tokens each, paged KV with block size 16 (the reference's choice for a mean
    prompt of 64..1024), at most 64 running sequences and 64 rows per step (the reference's
    max_batch). Decode-only steps replay a HIP graph per row count (captured before timing, as
    a server captures at start-up); steps with prefill rows launch eagerly; every step syncs once
    for its greedy tokens."""
    import importlib
    import numpy as np
    mf = importlib.import_module("llm_steadyinfer_amd.model_file")
    sch = importlib.import_module("llm_steadyinfer_amd.scheduler")
    bm = importlib.import_module("llm_steadyinfer_amd.batch_model")
    cfg = mf.LLAMA3_8B
    dev = lm_head[0].device
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed + 77)
    w = {"qkv": weights["qkv"], "o": weights["o"], "gu": weights["gate_up"],
         "down": weights["down"], "cls": lm_head,
         "emb": torch.randn((cfg.vocab, cfg.dim), generator=gen, device=dev),
         "norm": [torch.ones(cfg.dim, device=dev) for _ in range(2 * cfg.layer_num + 1)]}
    rng = np.random.default_rng(seed)
    lens = np.clip(np.rint(np.exp(rng.normal(np.log(200.0), sigma, n_seqs))), 16, 2048)
    prompts = [rng.integers(0, cfg.vocab, int(n)).tolist() for n in lens]
    max_seq = int(lens.max()) + n_new
    block = sch.Scheduler.resolve_block_size(float(lens.mean()))
    num_blocks = 64 * ((max_seq + block - 1) // block)  # 64 full-length sequences
    s = sch.Scheduler(None, max_batch=64, max_seq_len=max_seq, max_gen_len=n_new,
                      block_size=block, num_blocks=num_blocks)
    if native_model:  # model::PagedBatchModel (C++): the scheduler calls it with no Python
        nat = importlib.import_module("llm_steadyinfer_amd.native_scheduler")
        model = nat.NativePagedBatchModel(cfg, w, GS, max_rows=64, max_seq_len=max_seq,
                                          num_blocks=num_blocks, block_size=block, device=dev,
                                          packed=packed)
        native = True
    else:
        model = bm.PagedBatchModel(cfg, w, GS, max_rows=64, max_seq_len=max_seq,
                                   num_blocks=num_blocks, block_size=block, device=dev,
                                   packed=packed)
    # Decode-step graphs for every row count, captured at start-up (not timed).
    capture_s = model.capture_decode_graphs()
    if native:  # the C++ scheduler (scheduler::Scheduler), the model called back per step
        nat = importlib.import_module("llm_steadyinfer_amd.native_scheduler")
        s = nat.NativeScheduler(model, max_batch=64, max_seq_len=max_seq, max_gen_len=n_new,
                                block_size=block, num_blocks=num_blocks)
    else:
        s.forward = model.forward
    for p in ([5, 6, 7], [8, 9]):          # warm-up requests (every kernel once), not timed
        s.add_request(p)
    s.run()
    warm = {q.id for q in s.finished}
    steps0, rows0, pre0 = s.steps, s.rows_run, s.preemptions
    for p in prompts:
        s.add_request(p)
    torch.cuda.synchronize()
    # Step loop with the KV occupancy sampled before every step, as the reference's offline
    # benchmark does (benchmark/offline_batch_benchmark.cpp:240-268; host-side reads only).
    used_sum = alloc_sum = busy_sum = samples = peak_busy = 0
    t0 = time.perf_counter()
    while not s.all_finished():
        busy, used, alloc = s.kv_snapshot()
        if busy > 0:
            used_sum += used
            alloc_sum += alloc
            busy_sum += busy
            peak_busy = max(peak_busy, busy)
            samples += 1
        s.step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    done = [q for q in s.finished if q.id not in warm]
    gen_tokens = sum(len(q.generated_tokens) for q in done)
    # Per-request latencies as the reference's offline benchmark computes them
    # (benchmark/offline_batch_benchmark.cpp:280-324): TTFT = first token - admission, E2E =
    # finish - admission, TPOT = (E2E - TTFT) / (tokens - 1), ITL = the gaps between tokens;
    # nearest-rank percentiles (bench_common.h:95-101).
    def pct(v, p):
        if not v:
            return 0.0
        v = sorted(v)
        return v[min(len(v) - 1, max(0, int(np.ceil(p / 100.0 * len(v))) - 1))]
    ttft = [(q.first_token_time - q.admit_time) * 1e3 for q in done if q.generated_tokens]
    e2e = [(q.finish_time - q.admit_time) * 1e3 for q in done if q.generated_tokens]
    tpot = [(e - t) / (len(q.generated_tokens) - 1) for q, t, e in
            zip([q for q in done if q.generated_tokens], ttft, e2e)
            if len(q.generated_tokens) > 1]
    itl = [g for q in done for g in q.token_timestamps_ms]
    mean = lambda v: float(np.mean(v)) if v else 0.0
    latency = {"ttft_avg_ms": round(mean(ttft), 2), "ttft_p50_ms": round(pct(ttft, 50), 2),
               "ttft_p99_ms": round(pct(ttft, 99), 2), "tpot_avg_ms": round(mean(tpot), 3),
               "tpot_p50_ms": round(pct(tpot, 50), 3), "tpot_p99_ms": round(pct(tpot, 99), 3),
               "itl_avg_ms": round(mean(itl), 3), "itl_p99_ms": round(pct(itl, 99), 3),
               "e2e_avg_ms": round(mean(e2e), 1), "e2e_p99_ms": round(pct(e2e, 99), 1)}
    util = used_sum / alloc_sum if alloc_sum else 0.0
    kv = {"kv_cache_util_global": round(util, 4), "kv_cache_frag_global": round(1 - util, 4),
          "kv_cache_frag_per_seq": round(mean([1 - (len(q.prompt_tokens) +
                                                    len(q.generated_tokens)) / max_seq
                                               for q in done]), 4),
          "avg_busy_kv_slots": round(busy_sum / samples, 2) if samples else 0.0,
          "peak_busy_kv_slots": peak_busy}
    prompt_tokens = int(lens.sum())
    return {"workload": f"config 5: Llama-3-8B-shaped random-init INT8 model, {n_seqs} sequences, "
                        f"lognormal prompts (median 200, sigma {sigma}, clipped 16..2048; "
                        f"mean {lens.mean():.0f}, max {int(lens.max())}), {n_new} greedy tokens "
                        f"each, paged KV block {block}, max_batch 64" +
                        (", packed weights" if packed else ""),
            "output_tokens_per_s": round(gen_tokens / wall, 1), "latency": latency,
            "kv_cache": kv,
            "total_tokens_per_s": round((gen_tokens + prompt_tokens) / wall, 1),
            "wall_s": round(wall, 3), "generated_tokens": gen_tokens,
            "prompt_tokens": prompt_tokens, "steps": s.steps - steps0,
            "rows": s.rows_run - rows0, "preemptions": s.preemptions - pre0,
            "scheduler": "native (C++ scheduler::Scheduler)" if native else "python",
            "model": "native (C++ model::PagedBatchModel)" if native_model else "python",
            "kv_pool_GB": round(2 * 4 * cfg.layer_num * cfg.kv_dim * block * num_blocks / 1e9,
                                2),
            "graph_replays": model.graph_replays, "graph_capture_s": round(capture_s, 2),
            "launch": "decode-only steps: one HIP graph per row count (captured at start-up); "
                      "steps with prefill rows: eager; one host sync per step"}

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--packed", action="store_true",
                    help="also time the 1-64-row sweep and config 5 on packed weights "
                         "(sq8_pack_weights)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-batch", action="store_true", help="skip config 5 (continuous batching)")
    ap.add_argument("--native-scheduler", action="store_true",
                    help="config 5 on the C++ scheduler (scheduler::Scheduler) instead of the "
                         "Python one")
    ap.add_argument("--native-model", action="store_true",
                    help="config 5 on the C++ scheduler and the C++ batch model (no Python in "
                         "the step loop)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--graph", action="store_true", help="replay the step as one HIP graph")
    ap.add_argument("--profile", action="store_true",
                    help="short run for counter collection: a 256 MiB copy, then 5 decode steps")
    ap.add_argument("--profile-decode-gemm", action="store_true",
                    help="short run for counter collection: the four projections at M = 8, 32 "
                         "and 64 (configs 2), 3 launches each on distinct layers")
    ap.add_argument("--no-ceiling", action="store_true",
                    help="skip the read-probe and copy ceilings at the projections' sizes")
    ap.add_argument("--no-llama-decode", action="store_true",
                    help="skip the Llama-3-8B batch-1 end-to-end decode")
    ap.add_argument("--profile-prefill", action="store_true",
                    help="short run for counter collection: the four config-3 prefill GEMMs "
                         "(M = 2048), 3 launches each")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path. The matmul "
              "would shard column-parallel by output rows (qkv, gate/up, lm_head) and "
              "row-parallel by 64-aligned K groups (o, down) with one all-reduce.", file=sys.stderr)
        sys.exit(2)

    import torch
    sq8 = load_pkg()
    sq8.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(dev)  # default priority
    torch.cuda.set_stream(stream)
    ws = sq8.Workspace(dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(5678)

    t_init = time.perf_counter()
    weights = {p: [make_q8(torch, N, K, gen, dev) for _ in range(LAYERS)] for p, (N, K) in PROJ.items()}
    lm_head = make_q8(torch, VOCAB, HIDDEN, gen, dev)
    torch.cuda.synchronize()
    print(f"# weights ready in {time.perf_counter() - t_init:.1f}s", file=sys.stderr, flush=True)

    xgen = torch.Generator(device=dev)
    xgen.manual_seed(1234)

    def xbuf(M, K):
        return torch.randn((M, K), generator=xgen, device=dev, dtype=torch.float32)

    # ---------------------------------------------------------------- decode step (M = 1)
    xin = {p: xbuf(1, K) for p, (N, K) in PROJ.items()}
    yout = {p: torch.empty((1, N), device=dev) for p, (N, K) in PROJ.items()}
    calls = []
    for l in range(LAYERS):
        for p in PROJ:
            q, s = weights[p][l]
            calls.append(Call(sq8, xin[p], q, s, yout[p], stream, ws))
    x_head, y_head = xbuf(1, HIDDEN), torch.empty((1, VOCAB), device=dev)
    calls.append(Call(sq8, x_head, lm_head[0], lm_head[1], y_head, stream, ws))
    step_bytes = sum(c.bytes for c in calls)

    def step():
        for c in calls:
            c()

    if args.profile_prefill:
        a = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        b.copy_(a)
        for p, (N, K) in PROJ.items():
            x, y = xbuf(2048, K), torch.empty((2048, N), device=dev)
            for l in range(3):
                Call(sq8, x, *weights[p][l], y, stream, ws)()
            torch.cuda.synchronize()
        print(json.dumps({"profile_run": "prefill", "M": 2048, "launches_per_shape": 3}))
        return

    if args.profile_decode_gemm:
        a = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        b.copy_(a)
        # With --packed, the same calls on packed weights (repacked before the calls; the repack
        # launches are pack_weights_kernel in the trace).
        wts = ({p: [(sq8.pack_weights(q), s) for q, s in weights[p][:3]] for p in PROJ}
               if args.packed else weights)
        torch.cuda.synchronize()
        for M in (8, 32, 64):
            for p, (N, K) in PROJ.items():
                x, y = xbuf(M, K), torch.empty((M, N), device=dev)
                for l in range(3):
                    Call(sq8, x, *wts[p][l], y, stream, ws)()
                torch.cuda.synchronize()
        print(json.dumps({"profile_run": "decode_gemm", "M": [8, 32, 64],
                          "launches_per_shape": 3, "packed": bool(args.packed)}))
        return

    if args.profile:
        # Calibration copy of known size for FETCH_SIZE / WRITE_SIZE, then a few decode steps.
        a = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
        for _ in range(5):
            step()
        torch.cuda.synchronize()
        print(json.dumps({"profile_run": True, "launches_per_step": len(calls),
                          "step_algo_bytes": step_bytes}))
        return

    def timed(fn, steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps

    for _ in range(args.warmup):
        step()
    dt_eager = timed(step, args.steps)
    dt_graph = None
    if args.graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            step()
        for _ in range(args.warmup):
            graph.replay()
        dt_graph = timed(graph.replay, args.steps)
    dt = dt_graph if args.graph else dt_eager
    value = step_bytes / dt / 1e9

    # Average launch duration of the dominant kernel (the M=1 decode GEMV: every launch of the
    # step) from HIP events on the stream the kernels run on, around further eager steps.
    reps = max(3, args.steps // 2)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    step_launch_us = e0.elapsed_time(e1) * 1e3 / (reps * len(calls))
    launch_us = step_launch_us
    bytes_per_launch = step_bytes / len(calls)
    achieved = bytes_per_launch / launch_us / 1e3
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": round(bytes_per_launch * GEMV_TRAFFIC_RATIO),
                "kernel": "sq8 sweep_kernel, M=1 decode GEMV (per-shape configurations: "
                          "csrc/sq8_gemv.hip launch_stream)",
                "avg_launch_us": round(launch_us, 3),
                "avg_launch_us_source": "HIP events around whole eager steps / launches (the "
                                        "launches run back to back; the kernel trace in "
                                        "profiles/ gives the per-kernel durations)",
                "algo_bytes_per_launch": round(bytes_per_launch)}

    # The sections after the headline metric report an exception as {"error": ...} in their
    # field (traceback on stderr) instead of losing the whole line.
    def section(name, fn):
        try:
            return fn()
        except Exception as e:  # noqa: BLE001 - reported in the output line
            import traceback
            traceback.print_exc()
            print(f"# {name} failed: {e!r}", file=sys.stderr, flush=True)
            return {"error": f"{type(e).__name__}: {e}"}

    def tps(r, key):
        return r.get(key) if r else None

    # ---------------------------------------------------------------- configs 2 and 3 sweep
    sweep = []
    sweep_error = None

    def run_sweep():
        if not args.no_sweep:
            for M in (1, 8, 32, 64, 2048):
                for p, (N, K) in PROJ.items():
                    x, y = xbuf(M, K), torch.empty((M, N), device=dev)
                    reps = LAYERS if M <= 64 else 4
                    cs = [Call(sq8, x, *weights[p][l % LAYERS], y, stream, ws)
                          for l in range(reps)]
                    cs[0]()
                    a = torch.cuda.Event(enable_timing=True)
                    b = torch.cuda.Event(enable_timing=True)
                    a.record(stream)
                    for c in cs:
                        c()
                    b.record(stream)
                    torch.cuda.synchronize()
                    us = a.elapsed_time(b) * 1e3 / reps
                    tflops = cs[0].flops / us / 1e6
                    rec = {"proj": p, "M": M, "N": N, "K": K, "path": sq8.path_name(M, N, K, GS),
                           "us": round(us, 2), "GB/s": round(cs[0].bytes / us / 1e3, 1),
                           "TFLOP/s": round(tflops, 2)}
                    if sq8.path_name(M, N, K, GS) == "mfma":
                        # the f16 MFMA path issues two products (hi and lo) per useful multiply-add
                        rec["mfma_frac"] = round(2 * tflops / MFMA_F16_PEAK_TFLOPS, 4)
                    sweep.append(rec)
                    del x, y, cs
                print(f"# sweep M={M} done", file=sys.stderr, flush=True)

    try:
        run_sweep()
    except Exception as e:  # noqa: BLE001 - reported in the output line
        import traceback
        traceback.print_exc()
        sweep_error = f"{type(e).__name__}: {e}"

    # Config 3 (prefill, M = 2048): the GEMM is MFMA-bound. Issued f16 MFMA work is twice the
    # useful multiply-adds (hi and lo activation halves); peak = dense f16 MFMA.
    prefill = None
    pre = [r for r in sweep if r["M"] == 2048]
    if pre:
        us = sum(r["us"] for r in pre)
        flops = sum(2 * r["M"] * r["N"] * r["K"] for r in pre)
        useful = flops / us / 1e6
        prefill = {"bound": "mfma", "achieved": round(2 * useful, 1),
                   "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                   "frac": round(2 * useful / MFMA_F16_PEAK_TFLOPS, 4),
                   "useful_TFLOP/s": round(useful, 1),
                   "kernel": "sq8 gemm_kernel<2,4,2,2,3> (128x256 tiles, LDS-DMA ring), "
                             "M=2048 over the four Llama-3-8B projections",
                   "us_per_layer": round(us, 1)}

    # Streaming ceilings at each projection's size, against the GEMV's per-shape time (the M=1
    # rows of the sweep: 32 back-to-back launches of the shape).
    shape_bytes = [(p, algo_bytes(1, N, K)) for p, (N, K) in PROJ.items()] + \
        [("lm_head", algo_bytes(1, VOCAB, HIDDEN))]
    rceil = cceil = None
    if not args.no_ceiling:
        ceil = section("ceilings", lambda: (read_ceiling(torch, sq8, dev, shape_bytes),
                                            copy_ceiling(torch, dev, shape_bytes)))
        if isinstance(ceil, tuple):
            rceil, cceil = ceil
        else:
            roofline["read_ceiling"] = ceil
    if rceil is not None:
        gemv_us = {r["proj"]: r["us"] for r in sweep if r["M"] == 1}
        counts = {p: LAYERS for p in PROJ}
        counts["lm_head"] = 1
        per_shape = {}
        for p, nb in shape_bytes:
            rec = {"algo_bytes": nb, "read_probe_us": rceil[p]["us"], "copy_us": cceil[p]["us"],
                   "read_probe_setting": [rceil[p]["workgroups_per_cu"],
                                          rceil[p]["chunks_per_lane"]]}
            if p in gemv_us:
                rec["gemv_us"] = gemv_us[p]
                rec["gemv_GBps"] = round(nb / gemv_us[p] / 1e3, 1)
                rec["gemv_frac_of_peak"] = round(nb / gemv_us[p] / 1e3 / HBM_PEAK_GBS, 4)
                rec["gemv_frac_of_read_probe"] = round(rceil[p]["us"] / gemv_us[p], 3)
            per_shape[p] = rec
        ceil_step_us = sum(rceil[p]["us"] * counts[p] for p in counts)
        roofline["read_ceiling"] = {
            "step_ms": round(ceil_step_us / 1e3, 4),
            "frac_of_peak": round(step_bytes / ceil_step_us / 1e3 / HBM_PEAK_GBS, 4),
            "note": "the step's 129 launches priced at the read-only probe's time for each size",
            "per_shape": per_shape}

    llama = None
    if not args.no_llama_decode:
        llama = section("llama decode", lambda: llama_decode_run(torch, weights, lm_head))
        print(f"# llama decode done: {tps(llama, 'tokens_per_s')} tokens/s", file=sys.stderr,
              flush=True)

    decode = None
    if not args.no_decode:
        decode = section("decode", lambda: decode_run(torch))
        print(f"# decode done: {tps(decode, 'tokens_per_s')} tokens/s", file=sys.stderr,
              flush=True)

    # The same 1-64-row shapes on packed weights (one repack per layer's weight).
    sweep_packed = []
    if args.packed and not args.no_sweep:
        pw = {p: [(sq8.pack_weights(q), s_) for q, s_ in weights[p]] for p in PROJ}
        for M in (1, 8, 32, 64):
            for p, (N, K) in PROJ.items():
                x, y = xbuf(M, K), torch.empty((M, N), device=dev)
                cs = [Call(sq8, x, *pw[p][l], y, stream, ws) for l in range(LAYERS)]
                cs[0]()
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record(stream)
                for c in cs:
                    c()
                b.record(stream)
                torch.cuda.synchronize()
                us = a.elapsed_time(b) * 1e3 / LAYERS
                sweep_packed.append({"proj": p, "M": M, "N": N, "K": K, "us": round(us, 2),
                                     "GB/s": round(cs[0].bytes / us / 1e3, 1)})
                del x, y, cs
        del pw
        print("# packed sweep done", file=sys.stderr, flush=True)

    batch = None
    if not args.no_batch:
        batch = section("batch", lambda: batch_run(torch, weights, lm_head,
                                                   native=args.native_scheduler,
                                                   native_model=args.native_model))
        print(f"# batch done: {tps(batch, 'output_tokens_per_s')} output tokens/s",
              file=sys.stderr, flush=True)
    batch_packed = None
    if args.packed and not args.no_batch:
        batch_packed = section("packed batch", lambda: batch_run(
            torch, weights, lm_head, packed=True, native=args.native_scheduler,
            native_model=args.native_model))
        print(f"# packed batch done: {tps(batch_packed, 'output_tokens_per_s')} output "
              "tokens/s", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu:
        cpu = section("cpu baseline", lambda: cpu_baseline(torch, weights, args.cpu_seconds))

    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(dt * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8w_f32",
        "data": "synthetic (random-init N(0,0.02) weights, group-64 absmax INT8; x ~ N(0,1))",
        "config": {"workload": "Llama-3-8B INT8 decode matmuls, batch 1: 32 x (qkv 6144x4096, "
                               "o 4096x4096, gate_up 28672x4096, down 4096x14336) + lm_head "
                               "128256x4096, group 64", "global_batch": 1, "parallelism": "none"},
        "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        "launch": "hip_graph" if args.graph else "eager",
        "graph_GBps": round(step_bytes / dt_graph / 1e9, 1) if dt_graph else None,
        "decode_matmul_tokens_per_s": round(1.0 / dt, 1),
        "llama_decode_tokens_per_s": tps(llama, "tokens_per_s"),
        "llama_decode": llama,
        "decode_tokens_per_s": tps(decode, "tokens_per_s"),
        "decode": decode,
        "batch_output_tokens_per_s": tps(batch, "output_tokens_per_s"),
        "batch": batch,
        "batch_packed": batch_packed,
        "step_algo_bytes": step_bytes,
        "roofline": roofline,
        "prefill_roofline": prefill,
        "cpu_baseline": cpu,
        "sweep": sweep,
        "sweep_packed": sweep_packed or None,
        "sweep_error": sweep_error,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
