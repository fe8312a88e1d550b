"""The native scheduler (scheduler::Scheduler in libsq8_op.so, through native_scheduler.py)
against the Python restatement (scheduler.py), on the CPU with a fake model.

The fake model stores, at each row's (physical block, offset), a value chained from the value at
position - 1 read back through the row's block table (as a transformer's KV depends on every
earlier token), checks that no row writes into a block another row also references, and returns
a decode row's stored value as its token. Both schedulers must hand it the same rows and block
tables at every step of randomised workloads (staggered arrivals, pools small enough to preempt,
shared prefixes, stop tokens), end with the same tokens and counters, and return every block."""
import importlib

import numpy as np
import pytest

from conftest import load_pkg

load_pkg()
Scheduler = importlib.import_module("llm_steadyinfer_amd.scheduler").Scheduler
native = importlib.import_module("llm_steadyinfer_amd.native_scheduler")
NativeScheduler = native.NativeScheduler


class ChainModel:
    def __init__(self, block_size):
        self.bs = block_size
        self.kv = {}
        self.log = []
        self.ref = None  # block -> reference count, set once the scheduler exists

    def __call__(self, rows, tables):
        self.log.append([(r.seq.id, bool(r.is_decode), int(r.token), int(r.position), tuple(t))
                         for r, t in zip(rows, tables)])
        for r, t in zip(rows, tables):
            blk = t[r.position // self.bs]
            assert blk >= 0, "position beyond the row's blocks"
            assert self.ref(blk) == 1, f"write into shared block {blk}"
            prev = self.kv[(t[(r.position - 1) // self.bs], (r.position - 1) % self.bs)] \
                if r.position > 0 else 17
            self.kv[(blk, r.position % self.bs)] = (prev * 1000033 + r.token * 31 +
                                                    r.position) % 998244353
        return [self.kv[(t[r.position // self.bs], r.position % self.bs)] % 5000
                for r, t in zip(rows, tables) if r.is_decode]


def drive(kind, script, max_steps=3000, **kw):
    """script: list of (step index, prompts) arrivals. Returns the model's call log, the final
    tokens by id, the counters and the scheduler. A pool too small for the running set can cycle
    through eviction and resumption without end: such a run stops after max_steps steps."""
    model = ChainModel(kw["block_size"])
    cls = Scheduler if kind == "python" else NativeScheduler
    s = cls(model, **kw)
    model.ref = (lambda b: s.alloc.ref[b]) if kind == "python" else s.block_ref
    pending = sorted(script, key=lambda a: a[0])
    step = 0
    while pending or not s.all_finished():
        while pending and pending[0][0] <= step:
            for p in pending.pop(0)[1]:
                s.add_request(p)
        if s.all_finished():
            step += 1
            continue
        s.step()
        step += 1
        if step >= max_steps:
            break
    toks = {q.id: list(q.generated_tokens) for q in s.finished}
    counters = (s.steps, s.rows_run, s.preemptions, s.shared_prefix_blocks)
    return model.log, toks, counters, s


def workload(seed):
    rng = np.random.default_rng(seed)
    bs = int(rng.choice([4, 8, 16]))
    base = [int(t) for t in rng.integers(0, 5000, 64)]
    prompts = []
    for _ in range(int(rng.integers(4, 14))):
        n = int(rng.integers(1, 60))
        if rng.random() < 0.5:  # shares a prefix of base
            k = int(rng.integers(0, n + 1))
            p = base[:k] + [int(t) for t in rng.integers(0, 5000, n - k)]
        else:
            p = [int(t) for t in rng.integers(0, 5000, n)]
        prompts.append(p)
    arrivals = sorted(int(t) for t in rng.integers(0, 30, len(prompts)))
    script = [(a, [p]) for a, p in zip(arrivals, prompts)]
    max_gen = int(rng.integers(1, 24))
    max_seq = max(len(p) for p in prompts) + max_gen
    max_batch = int(rng.integers(1, 9))
    full = max_batch * ((max_seq + bs - 1) // bs)
    num_blocks = None if rng.random() < 0.3 else int(rng.integers(min(full, max(4, full // 4)),
                                                                     full + 1))
    stop = set(int(t) for t in rng.integers(0, 5000, int(rng.integers(0, 40))))
    kw = dict(max_batch=max_batch, max_seq_len=max_seq, max_gen_len=max_gen, block_size=bs,
              num_blocks=num_blocks, prefix_cache=bool(rng.random() < 0.7), stop_tokens=stop)
    return script, kw


@pytest.mark.parametrize("seed", range(60))
def test_native_equals_python_step_for_step(seed):
    script, kw = workload(seed)
    py = drive("python", script, **kw)
    nat = drive("native", script, **kw)
    assert len(nat[0]) == len(py[0])
    for i, (a, b) in enumerate(zip(nat[0], py[0])):
        assert a == b, f"step {i} differs"
    assert nat[1] == py[1]
    assert nat[2] == py[2]
    assert nat[3].invariant_holds()


def test_native_workloads_exercise_every_mechanism():
    """Across the seeds above, preemption, prefix sharing and stop tokens all occur."""
    pre = shared = stopped = 0
    for seed in range(60):
        script, kw = workload(seed)
        _, toks, (steps, rows, p, sh), s = drive("native", script, **kw)
        pre += p
        shared += sh
        stopped += sum(1 for t in toks.values() if t and t[-1] in kw["stop_tokens"])
        if s.all_finished():
            assert s.free_block_count() == (kw["num_blocks"] or
                                            kw["max_batch"] * -(-kw["max_seq_len"] //
                                                                kw["block_size"]))
    assert pre > 0 and shared > 0 and stopped > 0, (pre, shared, stopped)


def test_native_prefix_cache_never_shares_the_owners_last_prompt_block():
    """The owner's prompt is exactly two blocks; its prefill completes in step 0 and its first
    decode row (step 1) writes position 31 of block 1 again. A request admitted in step 1 mounts
    block 0 only (the chain model asserts that every written block is private)."""
    owner = list(range(100, 132))
    for kind in ("python", "native"):
        log, toks, (_, _, _, shared), _ = drive(
            kind, [(0, [owner]), (1, [owner + [7, 8, 9]])], max_batch=64, max_seq_len=60,
            max_gen_len=12, block_size=16, prefix_cache=True)
        assert len(log[0]) == 32 and log[1][0][1] and log[1][0][3] == 31
        assert shared == 1, kind


def test_native_forward_error_propagates_and_retires():
    def bad(rows, tables):
        raise ValueError("model failed")
    s = NativeScheduler(bad, max_batch=2, max_seq_len=32, block_size=4)
    s.add_request([1, 2, 3])
    with pytest.raises(ValueError, match="model failed"):
        s.step()
    assert s.all_finished() and s.free_block_count() == 16


def test_native_rejects_bad_arguments_and_requests():
    with pytest.raises(ValueError):
        NativeScheduler(lambda r, t: [], max_batch=0, max_seq_len=32)
    s = NativeScheduler(lambda r, t: [0] * sum(x.is_decode for x in r), max_batch=1,
                        max_seq_len=8, block_size=4)
    assert s.add_request([]) == -1
    assert s.add_request(list(range(8))) == -1  # leaves no room to generate
    assert s.add_request([1]) == 0


def test_native_run_bounds_steps():
    s = NativeScheduler(lambda r, t: [0] * sum(x.is_decode for x in r), max_batch=1,
                        max_seq_len=64, max_gen_len=50, block_size=4)
    s.add_request([1, 2])
    with pytest.raises(RuntimeError, match="no progress"):
        s.run(max_steps=3)


def test_cpp_scheduler_program_under_sanitizers(tmp_path):
    """tests/cpp/test_scheduler.cpp: 300 randomised workloads through scheduler::Scheduler with a
    C++ chain model, every sequence's tokens against its single-sequence run, built with g++
    -fsanitize=address,undefined (host code only)."""
    import shutil
    import subprocess
    from conftest import REPO
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    cpp = REPO / "llm-steadyinfer_amd" / "cpp"
    exe = tmp_path / "test_scheduler"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer",
           "-I", str(cpp / "include"), "-I", str(REPO / "tests" / "cpp"),
           str(REPO / "tests" / "cpp" / "test_scheduler.cpp")] + \
          [str(cpp / "src" / f) for f in ("scheduler.cpp", "block_allocator.cpp",
                                          "prefix_cache.cpp")] + ["-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-3000:]
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    print(res.stdout[-2000:])
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-3000:]
    assert "scheduler: 0 failure(s)" in res.stdout
