"""Host logic of the continuous-batching scheduler (llm-steadyinfer_amd/scheduler.py, restating
src/source/scheduler/scheduler.cpp and block_allocator.cpp), on the CPU with a fake model.

The fake model keeps a KV store addressed exactly like the paged cache: (physical block, offset)
from the row's block table. A row writes its token there; a decode row then hashes the tokens at
positions 0 .. pos of its own sequence (read back through its block table) into the next token.
Any block-table, chunking, ordering or recompute mistake changes the tokens, so every batched run
must reproduce the one-sequence-at-a-time run exactly."""
import importlib

import numpy as np
import pytest

from conftest import load_pkg

load_pkg()
sched_mod = importlib.import_module("llm_steadyinfer_amd.scheduler")
Scheduler, BlockAllocator = sched_mod.Scheduler, sched_mod.BlockAllocator


class FakeModel:
    def __init__(self, block_size):
        self.bs = block_size
        self.kv = {}
        self.calls = []

    def __call__(self, rows, tables):
        self.calls.append(rows)
        seen_prefill = False
        for r in rows:  # decode rows come first
            assert not (r.is_decode and seen_prefill), "decode rows must precede prefill rows"
            seen_prefill |= not r.is_decode
        for r, t in zip(rows, tables):  # every row writes before any row reads
            blk = t[r.position // self.bs]
            assert blk >= 0, "position beyond the row's blocks"
            self.kv[(blk, r.position % self.bs)] = r.token
        out = []
        for r, t in zip(rows, tables):
            if not r.is_decode:
                continue
            h = 1469598103
            for p in range(r.position + 1):
                h = (h * 1099511 + self.kv[(t[p // self.bs], p % self.bs)] + 7 * p) % 1000003
            out.append(h % 5000)
        return out


def run(prompts, max_batch, max_gen, block_size, num_blocks=None, max_seq=None):
    fake = FakeModel(block_size)
    max_seq = max_seq or max(len(p) for p in prompts) + max_gen
    s = Scheduler(fake, max_batch=max_batch, max_seq_len=max_seq, max_gen_len=max_gen,
                  block_size=block_size, num_blocks=num_blocks)
    ids = [s.add_request(p) for p in prompts]
    assert all(i >= 0 for i in ids)
    done = s.run(max_steps=20000)
    return {q.id: q.generated_tokens for q in done}, s, fake


def reference_tokens(prompts, max_gen, block_size):
    """One sequence at a time, whole prompt then token by token (no chunking limits)."""
    out = {}
    for i, p in enumerate(prompts):
        toks, _, _ = run([p], 1, max_gen, block_size)
        out[i] = toks[0]
    return out


PROMPTS = [list(np.random.default_rng(k).integers(0, 5000, n)) for k, n in
           enumerate([3, 17, 40, 9, 25, 1, 64, 33])]


def test_block_allocator_lifo_and_refcounts():
    a = BlockAllocator(num_blocks=8, num_rows=3, max_blocks_per_seq=4, block_size=16)
    r0 = a.allocate_blocks(2)
    r1 = a.allocate_blocks(3)
    assert (r0, r1) == (0, 1)
    assert a.table_row(0)[:2] == [0, 1] and a.table_row(1)[:3] == [2, 3, 4]
    assert a.append_blocks(0, 2) == 4 and a.table_row(0) == [0, 1, 5, 6]
    assert a.append_blocks(0, 1) == -1          # table row full
    assert a.allocate_blocks(2) == -1           # only 1 block left
    a.free_blocks_from(0, 2)                    # frees 5, 6 (pushed in order)
    assert a.free_block_count() == 3 and a.table_row(0) == [0, 1, -1, -1]
    assert a.allocate_blocks(1) == 2 and a.table_row(2)[0] == 6   # LIFO: last freed first
    for r in range(3):
        a.free_all(r)
    assert a.free_block_count() == 8 and all(c == 0 for c in a.ref)


def test_admission_rejects_prompt_without_room():
    s = Scheduler(lambda r, t: [], max_batch=2, max_seq_len=8, max_gen_len=4, block_size=4)
    assert s.add_request([1] * 8) == -1
    assert s.add_request([]) == -1
    i = s.add_request([1] * 6)
    assert i == 0 and s.waiting[0].max_gen_len == 2   # generation clamped to the cache


@pytest.mark.parametrize("max_batch,block_size", [(1, 4), (3, 4), (4, 16), (8, 8), (64, 16)])
def test_batched_tokens_equal_sequential(max_batch, block_size):
    ref = reference_tokens(PROMPTS, 10, block_size)
    got, s, fake = run(PROMPTS, max_batch, 10, block_size)
    assert got == ref
    assert s.alloc.free_block_count() == s.alloc.num_blocks and all(c == 0 for c in s.alloc.ref)
    assert all(len(v) == 10 for v in got.values())
    assert max(len(c) for c in fake.calls) <= max_batch


def test_chunked_prefill_mixes_with_decode():
    """With max_batch rows per step, long prompts prefill in chunks while earlier sequences
    decode in the same steps (decode rows first)."""
    got, s, fake = run(PROMPTS, 4, 10, 4)
    mixed = [c for c in fake.calls if any(r.is_decode for r in c) and
             any(not r.is_decode for r in c)]
    assert mixed, "no step mixed decode and prefill rows"
    assert got == reference_tokens(PROMPTS, 10, 4)


@pytest.mark.parametrize("num_blocks", [30, 35])
def test_preemption_recomputes_identically(num_blocks):
    """A pool far smaller than max_batch full sequences forces tail-block eviction; victims
    re-prefill (or keep their prefix) and still produce the sequential tokens."""
    ref = reference_tokens(PROMPTS, 12, 4)
    got, s, _ = run(PROMPTS, 4, 12, 4, num_blocks=num_blocks)
    assert s.preemptions > 0
    assert got == ref
    assert s.alloc.free_block_count() == num_blocks and all(c == 0 for c in s.alloc.ref)


@pytest.mark.parametrize("num_blocks", [19, 22, 25])
def test_exhausted_pool_finishes_with_correct_prefixes(num_blocks):
    """When a sequence cannot grow even after eviction it is finished early (as the reference
    does); what it generated is still a prefix of the sequential tokens, the run terminates and
    every block returns to the pool."""
    ref = reference_tokens(PROMPTS, 12, 4)
    got, s, _ = run(PROMPTS, 4, 12, 4, num_blocks=num_blocks)
    assert s.preemptions > 0
    for i, toks in got.items():
        assert toks == ref[i][:len(toks)]
    assert s.alloc.free_block_count() == num_blocks and all(c == 0 for c in s.alloc.ref)


def test_prefill_budget_levels():
    """Decode pressure moves the chunk budget one level per step within 512..4096."""
    s = Scheduler(lambda r, t: [0] * sum(1 for x in r if x.is_decode), max_batch=8,
                  max_seq_len=64, max_gen_len=4, block_size=4)
    for p in PROMPTS[:3]:
        s.add_request(p[:20])
    s.step()
    assert s.prefill_budget == 2048               # low pressure: 1024 -> 2048 toward 4096
    s.step()
    assert s.prefill_budget in (4096, 1024, 2048)
    assert 512 <= s.prefill_budget <= 4096


def test_resolve_block_size():
    assert Scheduler.resolve_block_size(10) == 8
    assert Scheduler.resolve_block_size(200) == 16
    assert Scheduler.resolve_block_size(2000) == 32


# ----------------------------------------------------------------------------- prefix cache, stop
class ChainModel(FakeModel):
    """Like FakeModel, but the value stored at position p depends on the value at p - 1 read back
    through the row's block table (as a transformer's KV depends on every earlier token), and no
    row may write into a block another row also references (shared prefix blocks are read-only).
    Rows of one sequence in a step come in position order, so p - 1 is always written first."""

    def __init__(self, block_size):
        super().__init__(block_size)
        self.alloc = None

    def __call__(self, rows, tables):
        self.calls.append(rows)
        for r, t in zip(rows, tables):
            blk = t[r.position // self.bs]
            assert blk >= 0, "position beyond the row's blocks"
            assert self.alloc.ref[blk] == 1, f"write into shared block {blk}"
            prev = self.kv[(t[(r.position - 1) // self.bs], (r.position - 1) % self.bs)] \
                if r.position > 0 else 17
            self.kv[(blk, r.position % self.bs)] = (prev * 1000033 + r.token * 31 + r.position) \
                % 998244353
        return [self.kv[(t[r.position // self.bs], r.position % self.bs)] % 5000
                for r, t in zip(rows, tables) if r.is_decode]


def run_chain(prompts, max_batch, max_gen, block_size, num_blocks=None, prefix=True, stop=(),
              max_seq=None, stagger=False):
    """Run the prompts; with stagger the first request runs alone until its prefill completes
    and the rest arrive then (entries exist only once an owner's prefill is done, and stay valid
    while the owner runs)."""
    fake = ChainModel(block_size)
    max_seq = max_seq or max(len(p) for p in prompts) + max_gen
    s = Scheduler(fake, max_batch=max_batch, max_seq_len=max_seq, max_gen_len=max_gen,
                  block_size=block_size, num_blocks=num_blocks, prefix_cache=prefix,
                  stop_tokens=stop)
    fake.alloc = s.alloc
    rest = prompts
    if stagger:
        assert s.add_request(prompts[0]) >= 0
        while not s.running or not s.running[0].prefill_complete:
            s.step()
        rest = prompts[1:]
    assert all(s.add_request(p) >= 0 for p in rest)
    done = s.run(max_steps=20000)
    return {q.id: q.generated_tokens for q in done}, s


def chain_reference(prompts, max_gen, block_size):
    return {i: run_chain([p], 1, max_gen, block_size, prefix=False)[0][0]
            for i, p in enumerate(prompts)}


_rng = np.random.default_rng(99)
BASE = [int(t) for t in _rng.integers(0, 5000, 40)]
OTHER = [int(t) for t in _rng.integers(0, 5000, 40)]
SHARED_PROMPTS = [
    BASE + [1, 2, 3],            # shares BASE's whole blocks with the next ones
    BASE + [4, 5, 6, 7, 8],
    BASE[:32],                   # a prefix exactly two blocks long (last block stays private)
    BASE[:16] + OTHER[16:40],    # block 1 differs after a shared block 0
    OTHER[:16] + BASE[16:40],    # block 1 equals BASE's block 1 after a different block 0
    BASE + [1, 2, 3],            # an exact repeat
    [9] * 5,
    BASE[:33],
]


@pytest.mark.parametrize("max_batch", [2, 3, 8])
def test_prefix_cache_tokens_equal_unshared(max_batch):
    ref = chain_reference(SHARED_PROMPTS, 30, 16)
    got, s = run_chain(SHARED_PROMPTS, max_batch, 30, 16, stagger=True)
    assert got == ref
    assert s.shared_prefix_blocks > 0
    assert s.alloc.free_block_count() == s.alloc.num_blocks and all(c == 0 for c in s.alloc.ref)
    assert len(s.prefix) > 0


def test_prefix_cache_skips_prefill_of_shared_blocks():
    """The rows run are fewer by exactly the shared positions, and the tokens are unchanged."""
    plain, s0 = run_chain(SHARED_PROMPTS, 8, 30, 16, prefix=False, stagger=True)
    shared, s1 = run_chain(SHARED_PROMPTS, 8, 30, 16, stagger=True)
    assert plain == shared
    # After the first prompt's prefill: BASE + [4..8] and the repeat share 2 blocks each,
    # BASE[:32] 1 (its last block stays private), BASE[:16] + OTHER 1, BASE[:33] 2,
    # OTHER[:16] + BASE[16:] and [9] * 5 none.
    assert s1.shared_prefix_blocks == 2 + 2 + 1 + 1 + 2
    assert s0.rows_run - s1.rows_run == 16 * s1.shared_prefix_blocks


def test_prefix_cache_is_off_by_default():
    _, s = run_chain(SHARED_PROMPTS, 8, 30, 16, prefix=False, stagger=True)
    assert s.prefix is None and s.shared_prefix_blocks == 0


def run_script(script, max_batch, max_gen, block_size, prefix=True):
    """Requests arrive in phases: each phase's prompts are added, then the scheduler steps until
    `until(s)` holds (a callable on the scheduler)."""
    fake = ChainModel(block_size)
    max_seq = max(len(p) for ps, _ in script for p in ps) + max_gen
    s = Scheduler(fake, max_batch=max_batch, max_seq_len=max_seq, max_gen_len=max_gen,
                  block_size=block_size, prefix_cache=prefix)
    fake.alloc = s.alloc
    for prompts, until in script:
        for p in prompts:
            assert s.add_request(p) >= 0
        while not until(s):
            s.step()
    s.run(max_steps=20000)
    return {q.id: q.generated_tokens for q in s.finished}, s


def prefilled(n):
    """Until the first n requests have completed their prefill (or finished)."""
    return lambda s: sum(1 for q in s.running + s.finished if q.prefill_complete or q.finished) \
        >= n


def test_prefix_cache_key_is_the_whole_prefix():
    """Owners X + Y and W + Z are both alive when X + Z arrives. Block 0 (X) matches the first
    owner; block 1 has Z's tokens, as the second owner's block 1 does, but that block's KV was
    computed after W: keyed by the whole prefix it does not match (keyed by the block's own
    tokens it would, and the chain model's tokens would change)."""
    X, Y, W, Z = (BASE[:16], BASE[16:32], OTHER[:16], OTHER[16:32])
    owners = [X + Y + [1, 2], W + Z + [3, 4]]
    late = [X + Z + [5, 6]]
    got, s = run_script([(owners, prefilled(2)), (late, lambda s: True)], 3, 30, 16)
    ref = chain_reference(owners + late, 30, 16)
    assert got == ref
    assert s.shared_prefix_blocks == 1  # only X


def test_prefix_cache_rejects_reallocated_block():
    """X = X0 + X1 + [1] and O = X0 + (200 tokens) run; X finishes holding 3 blocks and frees
    them. Y (33 tokens) takes X's row and, from the LIFO free list, X's blocks in reverse order,
    so X's block 1 is mounted again at index 1 of the same row, now holding Y's KV. C = X0 + X1
    + [...] then finds block 0 in O (valid) and, for block 1, X's entry: the block is referenced
    and mounted at the recorded (row, index), but it is another allocation of it. The
    per-allocation counter rejects it (without it the chain model's tokens change)."""
    X0, X1 = BASE[:16], BASE[16:32]
    long_tail = [int(t) for t in np.random.default_rng(5).integers(0, 5000, 200)]
    X, O, Y, C = X0 + X1 + [1], X0 + long_tail, OTHER[:33], X0 + X1 + [5, 6]
    x_done = lambda s: any(q.id == 0 for q in s.finished)
    got, s = run_script([([X, O], x_done), ([Y], prefilled(3)), ([C], lambda s: True)], 4, 12,
                        16)
    assert got == chain_reference([X, O, Y, C], 12, 16)
    assert s.shared_prefix_blocks == 1  # block 0 from O only


@pytest.mark.parametrize("num_blocks", [14, 16, 18, 20])
def test_prefix_cache_survives_preemption(num_blocks):
    """Pools too small for the running set: sequences holding shared blocks are cut back and
    resumed (or finished early when they cannot grow); every sequence's tokens are a prefix of
    its unshared run and every reference is returned."""
    ref = chain_reference(SHARED_PROMPTS, 24, 8)
    got, s = run_chain(SHARED_PROMPTS, 4, 24, 8, num_blocks=num_blocks, stagger=True)
    assert s.preemptions > 0 and s.shared_prefix_blocks > 0
    for i, toks in got.items():
        assert toks == ref[i][:len(toks)], i
    assert s.alloc.free_block_count() == num_blocks and all(c == 0 for c in s.alloc.ref)


def test_stop_tokens_retire_sequences():
    ref = chain_reference(PROMPTS, 12, 4)
    stop = {ref[0][3], ref[5][6]}
    got, s = run_chain(PROMPTS, 4, 12, 4, prefix=False, stop=stop)
    for i, toks in got.items():
        cut = next((k + 1 for k, t in enumerate(ref[i]) if t in stop), len(ref[i]))
        assert toks == ref[i][:cut], i
    assert len(got[0]) == 4


def test_block_allocator_shared_prefix_rows():
    a = BlockAllocator(num_blocks=6, num_rows=3, max_blocks_per_seq=4, block_size=4)
    r0 = a.allocate_blocks(3)                  # blocks 0, 1, 2
    r1 = a.allocate_blocks(0)                  # a row with no blocks yet is still taken
    assert (r0, r1) == (0, 1) and a.allocate_blocks(1) == 2
    assert a.append_blocks(r1, 1) == 1          # its own block first ...
    assert a.reserve_shared_prefix(r1, [0, 1])  # ... then the shared ones mounted in front
    assert a.table_row(r1) == [0, 1, 4, -1] and a.ref[0] == a.ref[1] == 2
    assert not a.reserve_shared_prefix(r1, [0, 1, 2])  # would overflow the row
    a.free_all(r0)
    assert a.ref[0] == a.ref[1] == 1 and a.ref[2] == 0 and 2 in a.free
    a.free_all(r1)
    a.free_all(2)
    assert a.free_block_count() == 6 and all(c == 0 for c in a.ref)


def test_prefix_cache_never_shares_the_owners_last_prompt_block():
    """An owner whose prompt fills exactly two blocks re-runs its last prompt token as its first
    decode row, writing position 31 of block 1 again. A request admitted in that same step must
    not mount block 1 (the chain model asserts every written block is private), only block 0."""
    owner = BASE[:32]
    late = BASE[:32] + [7, 8, 9]
    prefill_done = lambda s: any(q.prefill_complete for q in s.running)
    got, s = run_script([([owner], prefill_done), ([late], lambda s: True)], 2, 12, 16)
    assert got == chain_reference([owner, late], 12, 16)
    assert s.shared_prefix_blocks == 1
