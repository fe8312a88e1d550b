"""The native scheduler (scheduler::Scheduler in libsq8_op.so, through native_scheduler.py)
against the Python restatement (scheduler.py), on the CPU with a fake model.

The fake model stores, at each row's (physical block, offset), a value chained from the value at
position - 1 read back through the row's block table (as a transformer's KV depends on every
earlier token), checks that no row writes into a block another row also references, and returns
a decode row's stored value as its token. Both schedulers must hand it the same rows and block
tables at every step of randomised workloads (staggered arrivals, pools small enough to preempt,
shared prefixes, stop tokens), end with the same tokens and counters, and return every block."""
import ctypes
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


# A preemption inside the decode pass removes a prefill-incomplete victim that sits before the
# sequence being grown; the native scheduler once walked its running list by index after that
# list was rebuilt, so the sequence after the grown one lost its row for the step (this workload
# diverged from the Python scheduler at step 16 before the walk used a snapshot).
_EARLIER_VICTIM = (
    [(2, [[2631, 3399]]), (3, [[416, 216, 4989]]), (4, [[3126, 1574, 1094, 4025]]),
     (6, [[1132, 2054, 1253, 1919]]),
     (6, [[807, 3566, 3218, 3872, 4561, 4647, 4973, 4354, 4847, 4690]])],
    dict(max_batch=4, max_seq_len=28, max_gen_len=18, block_size=4, num_blocks=5,
         prefix_cache=False, stop_tokens=set()))


def test_native_keeps_rows_after_an_earlier_victim_is_preempted():
    script, kw = _EARLIER_VICTIM
    py = drive("python", script, max_steps=400, **kw)
    nat = drive("native", script, max_steps=400, **kw)
    assert py[2][2] > 0, "the workload must preempt"
    assert nat[0] == py[0]
    assert nat[1] == py[1] and nat[2] == py[2]
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


def test_native_model_binding_rejects_bad_configuration():
    """sq8_batch_model_create validates the configuration before touching the device."""
    import torch
    mf = importlib.import_module("llm_steadyinfer_amd.model_file")
    cfg = mf.ModelConfig(dim=256, hidden_dim=512, layer_num=1, head_num=3, kv_head_num=2,
                         vocab_size=-100, seq_len=64, rope_theta=1e4)  # 3 heads over 2 kv heads
    t = torch.zeros(16)
    w = {k: [(t, t)] for k in ("qkv", "o", "gu", "down")}
    w.update(cls=(t, t), emb=t, norm=[t, t, t])
    with pytest.raises(RuntimeError, match="model configuration"):
        native.NativePagedBatchModel(cfg, w, 64, max_rows=4, max_seq_len=64, num_blocks=16,
                                     block_size=4)


def test_native_scheduler_calls_a_native_forward_directly():
    """A model exposing native_forward (a C function with the callback's signature) is called
    from C++ with no Python in the loop; its failure surfaces as RuntimeError. Here the C
    function is sq8_batch_model_forward on a NULL model, which fails every call."""
    L = native.op_lib()
    native._bind_model(L)

    class Stub:
        native_forward = (ctypes.cast(L.sq8_batch_model_forward, ctypes.c_void_p).value, None)

        def last_error(self):
            return "stub failed"

    s = NativeScheduler(Stub(), max_batch=2, max_seq_len=32, block_size=4)
    assert s.add_request([1, 2, 3]) == 0
    with pytest.raises(RuntimeError, match="stub failed"):
        s.run(max_steps=10)
    assert s.all_finished() and s.free_block_count() == 16


# ----------------------------------------------------------------------------- native model calls
# Argument kinds of the logged libsq8 calls, in C order: p pointer, i integer, f float, s stream
# (not logged). Workspace sizes and the fused-epilogue rule restate tests/cpp/mock_sq8.cpp.
_SPEC = {
    "sq8_matmul_rmsnorm": "ppppfpppiiis",
    "sq8_matmul_rmsnorm_swiglu": "ppppfpppiiis",
    "sq8_rope_attention_decode": "piiippppppis",
    "sq8_rope_attention_decode_ws": "piiippppppipis",
    "sq8_argmax_advance": "pipipppiips",
    "sq8_step_advance": "ppps",
    "sq8_matmul": "ppppiiiipis", "sq8_matmul_packed": "ppppiiiipis",
    "sq8_matmul_epilogue": "ppppiiiiippis", "sq8_matmul_epilogue_packed": "ppppiiiiippis",
    "sq8_matmul_rmsnorm_rows": "pppfpppiiiiipis", "sq8_matmul_rmsnorm_rows_packed":
    "pppfpppiiiiipis", "sq8_embedding": "piipips", "sq8_rmsnorm": "pppiifs",
    "sq8_add_rmsnorm": "ppppiifs", "sq8_rope_tables": "ppiifs",
    "sq8_paged_rope_kv": "piiiippiipppps", "sq8_paged_attention": "piiiiippiippps",
    "sq8_paged_attention_ws": "piiiiippiippppis", "sq8_swiglu_rows": "piips",
    "sq8_argmax_rows": "piips"}


class _RecordingLib:
    """Logs libsq8 calls like tests/cpp/mock_sq8.cpp: a pointer as p<allocation id>[+<byte
    offset>], the allocation found among the tensors `sources()` returns as (tensor, owned)."""

    def __init__(self):
        self.log, self.ids, self.sources, self.allocs = [], {}, (lambda: []), []

    def _rescan(self):
        seen = {}
        for t, owned in self.sources():
            st = t.untyped_storage()
            seen[st.data_ptr()] = (st.nbytes(), owned)
        self.allocs = sorted((b, n, o) for b, (n, o) in seen.items())

    def _ptr(self, a):
        for attempt in range(2):
            for base, n, owned in self.allocs:
                if base <= a < base + n:
                    key = base
                    if key not in self.ids:
                        self.ids[key] = (len(self.ids) + 1, n, owned)
                    i = self.ids[key][0]
                    return f"p{i}" if a == base else f"p{i}+{a - base}"
            self._rescan()
        return "?"

    def alloc_lines(self):
        return [f"alloc p{i} {n}" for i, n, owned in sorted(self.ids.values()) if owned]

    def _fmt(self, name, args):
        out = [name]
        for kind, a in zip(_SPEC[name], args):
            if kind == "s":
                continue
            if kind == "p":
                if not a:
                    out.append("0")
                else:
                    out.append(self._ptr(int(a)))
            elif kind == "f":
                out.append("%.6g" % np.float32(a))
            else:
                out.append(str(int(a)))
        self.log.append(" ".join(out))
        return 0

    def __getattr__(self, name):
        if name in _SPEC:
            return lambda *a: self._fmt(name, a)
        if name in ("sq8_epilogue_fused", "sq8_epilogue_packed_fused"):
            return lambda M, N, K, gs: int(M > 4 and N % 2 == 0)
        if name in ("sq8_epilogue_workspace_bytes", "sq8_rmsnorm_rows_workspace_bytes"):
            return lambda *a: 4096
        if name in ("sq8_epilogue_packed_workspace_bytes",
                    "sq8_rmsnorm_rows_packed_workspace_bytes", "sq8_packed_workspace_bytes"):
            return lambda *a: 8192
        if name == "sq8_workspace_bytes":
            return lambda *a: 4096
        if name == "sq8_argmax_workspace_bytes":
            return lambda *a: 1024
        if name == "sq8_decode_attention_workspace_bytes":
            return lambda *a: 2048
        if name == "sq8_paged_attention_workspace_bytes":
            return lambda *a: 2048
        if name == "sq8_packed_weight_bytes":
            return lambda N, K: ((N + 15) // 16) * 16 * K
        if name == "sq8_pack_weights":
            return lambda *a: 0
        raise AttributeError(name)


def _tensors(model, weights):
    """(tensor, owned) for the model's own buffers (attributes, workspaces) and the weights."""
    import torch
    out = []
    if model is not None:
        for v in list(vars(model).values()):
            for t in (v, getattr(v, "buf", None)):
                if isinstance(t, torch.Tensor):
                    out.append((t, True))
        for v in getattr(model, "w", {}).values():
            items = v if isinstance(v, (list, tuple)) else [v]
            for it in items:
                for t in (it if isinstance(it, tuple) else (it,)):
                    t = getattr(t, "data", t) if not isinstance(t, torch.Tensor) else t
                    if isinstance(t, torch.Tensor):
                        out.append((t, False))
    for v in weights.values():
        for it in (v if isinstance(v, list) else [v]):
            for t in (it if isinstance(it, tuple) else (it,)):
                out.append((t, False))
    return out


def _script(rng):
    """Steps over a 40-block pool (blocks of 4, tables of 16): prefill-only, mixed,
    decode-only at several row counts (twice at the same count), up to 8 rows."""
    steps, pos_of = [], {}
    tables = {s: [int(b) for b in rng.permutation(40)[:16]] for s in range(8)}
    for B, nd in ((3, 0), (7, 2), (5, 5), (5, 5), (8, 3), (2, 2), (8, 8), (1, 0), (4, 4)):
        seqs = rng.choice(8, B, replace=nd == B)
        rows = []
        for i, sq in enumerate(seqs):
            p = pos_of.get(int(sq), 0)
            pos_of[int(sq)] = p + 1
            rows.append((int(rng.integers(0, 50)), min(p, 60), tables[int(sq)]))
        steps.append((B, nd, rows))
    return steps


def _python_log(steps, packed, split):
    import torch
    pkg = load_pkg()
    bm = importlib.import_module("llm_steadyinfer_amd.batch_model")
    mf = importlib.import_module("llm_steadyinfer_amd.model_file")
    rec = _RecordingLib()
    saved = (pkg.lib, bm.lib, pkg._check_matmul, pkg._check_paged, torch.cuda.current_stream)

    class _S:
        cuda_stream = 0
    try:
        pkg.lib = bm.lib = lambda: rec
        pkg._check_matmul = lambda *a, **k: None
        pkg._check_paged = lambda *a, **k: None
        torch.cuda.current_stream = lambda *a, **k: _S()
        cfg = mf.ModelConfig(dim=64, hidden_dim=96, layer_num=2, head_num=4, kv_head_num=2,
                             vocab_size=-50, seq_len=64, rope_theta=1e6)
        q = lambda n, k: (torch.zeros((n, k), dtype=torch.int8), torch.zeros(n * k // 64))
        w = {"qkv": [q(128, 64) for _ in range(2)], "o": [q(64, 64) for _ in range(2)],
             "gu": [q(192, 64) for _ in range(2)], "down": [q(64, 96) for _ in range(2)],
             "cls": q(50, 64), "emb": torch.zeros((50, 64)),
             "norm": [torch.ones(64) for _ in range(5)]}
        holder = {}
        rec.sources = lambda: _tensors(holder.get("m"), w)
        m = holder["m"] = bm.PagedBatchModel.__new__(bm.PagedBatchModel)
        m.__init__(cfg, w, 64, max_rows=8, max_seq_len=64, num_blocks=40, block_size=4,
                   device="cpu", use_graphs=False, split_kv=split, packed=packed)
        for B, nd, rows in steps:
            rec.log.append("step")
            m.forward_arrays(np.array([r[0] for r in rows], np.int32),
                             np.array([r[1] for r in rows], np.int32),
                             np.array([r[2] for r in rows], np.int32), nd)
    finally:
        pkg.lib, bm.lib, pkg._check_matmul, pkg._check_paged, torch.cuda.current_stream = saved
    return rec.log + rec.alloc_lines()


_EXE = {}


def _calls_exe(tmp_path):
    """The call-log program, compiled once per test session."""
    import shutil
    import subprocess
    from conftest import REPO
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    if "calls" in _EXE and _EXE["calls"].exists():
        return _EXE["calls"]
    exe = tmp_path / "test_batch_model_calls"
    _EXE["calls"] = exe
    if not exe.exists():
        cpp = REPO / "llm-steadyinfer_amd" / "cpp"
        t = REPO / "tests" / "cpp"
        cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
               "-fno-sanitize-recover=undefined", "-I", str(t / "mock_hip"), "-I",
               str(cpp / "include"), "-I", str(t), str(t / "test_batch_model_calls.cpp"),
               str(t / "mock_sq8.cpp"), str(cpp / "src" / "paged_batch_model.cpp"),
               str(cpp / "src" / "int8_decoder.cpp"), "-o", str(exe)]
        res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
        assert res.returncode == 0, res.stderr[-3000:]
    return exe


def _cpp_log(steps, packed, graphs, split, tmp_path, capture_first=False):
    import subprocess
    exe = _calls_exe(tmp_path)
    lines = [f"batch {int(packed)} {int(graphs)} {int(split)}"] + \
        (["capture"] if capture_first else [])
    for B, nd, rows in steps:
        lines.append(f"{B} {nd}")
        lines.append(" ".join(str(r[0]) for r in rows))
        lines.append(" ".join(str(r[1]) for r in rows))
        lines.append(" ".join(str(b) for r in rows for b in r[2]))
    res = subprocess.run([str(exe)], input="\n".join(lines) + "\n", capture_output=True,
                         text=True, timeout=120)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-3000:]
    return res.stdout.splitlines()


@pytest.mark.parametrize("packed,split", [(False, True), (False, False), (True, True)])
def test_native_model_issues_the_python_models_calls(tmp_path, packed, split):
    """model::PagedBatchModel (C++) and batch_model.PagedBatchModel (Python, GPU-tested) issue
    the same libsq8 calls with the same arguments and buffer roles for the same steps, eagerly:
    prefill-only, mixed and decode-only steps, fused and unfused epilogues, row-major or packed
    weights, with and without the split-KV workspace. The C++ side runs under ASan/UBSan."""
    steps = _script(np.random.default_rng(3))
    py = _python_log(steps, packed, split)
    cpp = _cpp_log(steps, packed, False, split, tmp_path)
    assert len(cpp) == len(py)
    for i, (a, b) in enumerate(zip(cpp, py)):
        assert a == b, f"call {i}: C++ {a!r} != Python {b!r}"


def test_native_model_graphs_replay_decode_steps(tmp_path):
    """With graphs, the first decode-only step at a row count runs eagerly and is captured (its
    launches appear twice); later decode-only steps at that count replay the graph; steps with
    prefill rows always run eagerly. capture_decode_graphs() captures every count up front."""
    steps = _script(np.random.default_rng(3))
    eager = _cpp_log(steps, False, False, True, tmp_path)
    log = _cpp_log(steps, False, True, True, tmp_path)
    def per_step(lg):
        counts = []
        for line in lg:
            if line == "step":
                counts.append(0)
            elif counts and not line.startswith("alloc "):
                counts[-1] += 1
        return counts
    e, g = per_step(eager), per_step(log)
    n = e[2]  # launches of one 5-row decode-only step
    assert g[2] == 2 * n and g[3] == 1  # eager + capture, then one graph launch
    assert g[0] == e[0] and g[1] == e[1]  # steps with prefill rows stay eager
    log = _cpp_log(steps, False, True, True, tmp_path, capture_first=True)
    g = per_step(log)
    assert g[2] == 1 and g[3] == 1 and g[6] == 1 and g[8] == 1


def test_capture_after_a_step_is_refused(tmp_path):
    """capture_decode_graphs runs placeholder rows that write K/V into block 0: after a step a
    sequence may hold that block, so both models refuse (C++ with an error, Python raising)."""
    import subprocess
    from types import SimpleNamespace
    steps = _script(np.random.default_rng(3))
    exe = _calls_exe(tmp_path)
    B, nd, rows = steps[0]
    lines = ["batch 0 1 1", f"{B} {nd}", " ".join(str(r[0]) for r in rows),
             " ".join(str(r[1]) for r in rows), " ".join(str(b) for r in rows for b in r[2]),
             "capture"]
    res = subprocess.run([str(exe)], input="\n".join(lines) + "\n", capture_output=True,
                         text=True, timeout=120)
    assert res.returncode != 0
    assert "capture failed: capture_decode_graphs after a forward step" in res.stdout
    bm = importlib.import_module("llm_steadyinfer_amd.batch_model")
    with pytest.raises(RuntimeError, match="after a forward step"):
        bm.PagedBatchModel.capture_decode_graphs(SimpleNamespace(rows_run=3))


def _python_decoder_log(prompt, n_new, split):
    import torch
    pkg = load_pkg()
    dec = importlib.import_module("llm_steadyinfer_amd.decoder")
    mf = importlib.import_module("llm_steadyinfer_amd.model_file")
    rec = _RecordingLib()
    saved = (pkg.lib, dec.lib, torch.cuda.current_stream, torch.cuda.synchronize)

    class _S:
        cuda_stream = 0
    try:
        pkg.lib = dec.lib = lambda: rec
        torch.cuda.current_stream = lambda *a, **k: _S()
        torch.cuda.synchronize = lambda *a, **k: None
        pkg._check_matmul_saved = pkg._check_matmul
        pkg._check_matmul = lambda *a, **k: None
        cfg = mf.ModelConfig(dim=64, hidden_dim=96, layer_num=2, head_num=4, kv_head_num=2,
                             vocab_size=-50, seq_len=64, rope_theta=1e6)
        q = lambda n, k: (torch.zeros((n, k), dtype=torch.int8), torch.zeros(n * k // 64))
        w = {"qkv": [q(128, 64) for _ in range(2)], "o": [q(64, 64) for _ in range(2)],
             "gu": [q(192, 64) for _ in range(2)], "down": [q(64, 96) for _ in range(2)],
             "cls": q(50, 64), "emb": torch.zeros((50, 64)),
             "norm": [torch.ones(64) for _ in range(5)]}
        holder = {}
        rec.sources = lambda: _tensors(holder.get("m"), w)
        d = holder["m"] = dec.Int8Decoder.__new__(dec.Int8Decoder)
        d.__init__(cfg, w, 64, 64, device="cpu")
        if not split:
            d.att_ws = None
        d.generate(prompt, n_new, use_graph=False)
    finally:
        pkg._check_matmul = pkg._check_matmul_saved
        pkg.lib, dec.lib, torch.cuda.current_stream, torch.cuda.synchronize = saved
    return rec.log + rec.alloc_lines()


def _cpp_decoder_log(prompt, n_new, graph, split, tmp_path):
    import subprocess
    exe = _calls_exe(tmp_path)
    inp = f"decoder {int(graph)} {int(split)} {n_new} {len(prompt)}\n" + \
        " ".join(map(str, prompt)) + "\n"
    res = subprocess.run([str(exe)], input=inp, capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-3000:]
    return res.stdout.splitlines()


@pytest.mark.parametrize("split", [True, False])
def test_native_decoder_issues_the_python_decoders_calls(tmp_path, split):
    """model::Int8Decoder (C++) and decoder.Int8Decoder (Python, GPU-tested) issue the same
    libsq8 calls for a 5-token prompt and 4 generated tokens (eager steps): the fused QKV / gate
    / up prologues with the residual stream ping-ponging, RoPE + attention in one launch, the
    classifier and argmax + advance + embedding, and the prompt steps' embedding and advance."""
    prompt = [3, 1, 4, 1, 5]
    py = _python_decoder_log(prompt, 4, split)
    cpp = _cpp_decoder_log(prompt, 4, False, split, tmp_path)
    assert len(cpp) == len(py)
    for i, (a, b) in enumerate(zip(cpp, py)):
        assert a == b, f"call {i}: C++ {a!r} != Python {b!r}"


def test_native_decoder_replays_one_graph_per_token(tmp_path):
    """With the graph: the prompt steps run eagerly, one step is captured (its launches logged
    once, not run), and each generated token is one graph launch."""
    eager = _cpp_decoder_log([3, 1, 4], 5, False, True, tmp_path)
    graph = _cpp_decoder_log([3, 1, 4], 5, True, True, tmp_path)
    assert graph.count("graph_launch") == 5
    steps_eager = sum(1 for l in eager if l.startswith("sq8_argmax_advance"))
    steps_graph = sum(1 for l in graph if l.startswith("sq8_argmax_advance"))
    assert steps_eager == 5 and steps_graph == 1


# ----------------------------------------------------------------------------- device weights
def _pack_ref(q):
    N, K = q.shape
    T, G = (N + 15) // 16, K // 64
    pad = np.zeros((T * 16, K), np.int8)
    pad[:N] = q
    return pad.reshape(T, 16, G, 4, 16).transpose(0, 2, 3, 1, 4).reshape(-1)


@pytest.mark.parametrize("vocab,packed", [(-300, False), (-300, True), (300, False)])
def test_device_weights_upload_layout(tmp_path, vocab, packed):
    """model::DeviceWeights (C++) uploads a model file (read by the C++ loader) as the fused
    weights the native models take: QKV = [wq; wk; wv], gate/up = [w1; w3] with scales
    concatenated, optionally in the packed layout, plus the embedding and the norms; equal byte
    for byte to the same layout built in numpy from the Python reader. vocab > 0 is the
    reference's tied layout. Built with g++ against host stand-ins of HIP and libsq8."""
    import shutil
    import subprocess
    from conftest import REPO
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    mf = importlib.import_module("llm_steadyinfer_amd.model_file")
    cfg = mf.ModelConfig(dim=128, hidden_dim=192, layer_num=2, head_num=4, kv_head_num=2,
                         vocab_size=vocab, seq_len=64, rope_theta=1e4)
    path = mf.write_random(tmp_path / "m.bin", cfg, 64, seed=5, w_std=0.1)
    exe = _EXE.get("weights") or tmp_path / "test_device_weights"
    cpp, t = REPO / "llm-steadyinfer_amd" / "cpp", REPO / "tests" / "cpp"
    srcs = [str(cpp / "src" / f"{f}.cpp") for f in ("alloc", "buffer", "tensor", "layer", "matmul",
                                                    "int8_model_file", "hip_config",
                                                    "device_weights")]
    if not exe.exists():
        res = subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
                              "-fno-sanitize-recover=undefined", "-I", str(t / "mock_hip"), "-I",
                              str(cpp / "include"), "-I", str(t),
                              str(t / "test_device_weights.cpp"), str(t / "mock_sq8.cpp")] +
                             srcs + ["-o", str(exe)], capture_output=True, text=True, timeout=300)
        assert res.returncode == 0, res.stderr[-3000:]
        _EXE["weights"] = exe
    out = tmp_path / "uploaded.bin"
    res = subprocess.run([str(exe), str(path), str(int(packed)), str(out)], capture_output=True,
                         text=True, timeout=120)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-3000:]
    m = mf.ModelFile(path)
    parts = []

    def fused(names, layer):
        qs, ss = zip(*(m.quant(n, layer) for n in names))
        q = np.concatenate(qs, axis=0)
        parts.append(_pack_ref(q) if packed else q.reshape(-1))
        parts.append(np.concatenate(ss).astype(np.float32).view(np.int8))
    for l in range(cfg.layer_num):
        fused(("wq", "wk", "wv"), l)
        fused(("wo",), l)
        fused(("w1", "w3"), l)
        fused(("w2",), l)
    fused(("cls",), 0)
    parts.append(np.asarray(m.fp32("embedding"), np.float32).reshape(-1).view(np.int8))
    for i in range(2 * cfg.layer_num + 1):
        parts.append(np.asarray(m.fp32("rmsnorm", i), np.float32).reshape(-1).view(np.int8))
    want = np.concatenate(parts)
    got = np.fromfile(out, np.int8)
    assert got.size == want.size and np.array_equal(got, want)
    assert res.stdout.splitlines()[0] == f"config 128 192 2 4 2 300 64"
    assert res.stdout.count("sq8_pack_weights") == (4 * cfg.layer_num + 1 if packed else 0)


def test_native_from_file_reports_a_missing_file(tmp_path):
    """The C++ file path fails cleanly (no device work) for a file that does not exist."""
    with pytest.raises(RuntimeError, match="native decoder"):
        native.NativeInt8Decoder.from_file(tmp_path / "missing.bin", max_seq=64)
    with pytest.raises(RuntimeError, match="native batch model"):
        native.NativePagedBatchModel.from_file(tmp_path / "missing.bin", 4, 64, 16, 4)


@pytest.mark.parametrize("kind", ["python", "native"])
def test_serving_timestamps(kind):
    """Per-request timestamps as the reference records them: arrival <= admission <= first
    token <= last token <= finish; one inter-token gap per generated token after the first, the
    gaps summing to last - first; one batch-reconstruct time per decode-only step."""
    import time as _t
    calls = []

    def model(rows, tables):
        _t.sleep(0.0005)
        calls.append(all(r.is_decode for r in rows))
        return [1] * sum(r.is_decode for r in rows)
    cls = Scheduler if kind == "python" else NativeScheduler
    s = cls(model, max_batch=3, max_seq_len=64, max_gen_len=6, block_size=4)
    for n in (5, 9, 2, 17):
        s.add_request(list(range(1, n + 1)))
    done = s.run(max_steps=1000)
    for q in done:
        assert q.arrival_time <= q.admit_time <= q.first_token_time <= q.last_token_time \
            <= q.finish_time, q.id
        assert len(q.token_timestamps_ms) == len(q.generated_tokens) - 1
        assert abs(sum(q.token_timestamps_ms) / 1e3 - (q.last_token_time - q.first_token_time)) \
            < 1e-6
        assert min(q.token_timestamps_ms) > 0.4  # each step sleeps 0.5 ms
    assert len(s.batch_reconstruct_times_ms) == sum(calls) > 0


def test_native_model_refuses_bad_rows_before_launching(tmp_path):
    """model::PagedBatchModel::forward_batch checks every row on the host (row counts, table
    width, position range, a cache block mapped for every position attended, token ids) and
    refuses with nothing launched: a bad table would otherwise become an out-of-bounds read."""
    import subprocess
    exe = _calls_exe(tmp_path)
    res = subprocess.run([str(exe)], input="validate\n", capture_output=True, text=True,
                         timeout=60)
    assert res.returncode == 0, res.stdout + res.stderr[-2000:]
    lines = res.stdout.splitlines()
    assert sum(1 for l in lines if ": " in l and "accepted" not in l) == 8
    calls = [l for l in lines if l.startswith("sq8_")]
    assert len(calls) == 1 and calls[0].startswith("sq8_rope_tables")  # init() only


def test_kv_snapshot_equal_in_both_schedulers():
    """The occupancy snapshot (busy rows, tokens held, tokens allocated) agrees between the two
    schedulers before every step of a preempting workload."""
    script, kw = workload(7)
    snaps = {}
    for kind in ("python", "native"):
        model = ChainModel(kw["block_size"])
        s = (Scheduler if kind == "python" else NativeScheduler)(model, **kw)
        model.ref = (lambda b: s.alloc.ref[b]) if kind == "python" else s.block_ref
        for _, ps in script:
            for p in ps:
                s.add_request(p)
        out = []
        while not s.all_finished() and len(out) < 3000:
            out.append(s.kv_snapshot())
            s.step()
        snaps[kind] = out
    assert snaps["python"] == snaps["native"] and len(snaps["python"]) > 10
