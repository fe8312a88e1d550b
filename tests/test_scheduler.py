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
