"""Continuous-batching scheduler with a paged KV block pool: the host bookkeeping of the
reference's Scheduler (src/source/scheduler/scheduler.cpp) and BlockAllocator
(src/source/scheduler/block_allocator.cpp), driving a batched model forward.

One step (Scheduler::step, scheduler.cpp:122-164):
  1. admission (try_admit_sequences, :170-262): waiting sequences become RUNNING while fewer than
     max_batch run; a fresh sequence gets a block-table row with its prompt's blocks, a preempted
     one resumes with the blocks it kept. When the pool is short, tail blocks of the most recently
     admitted running sequences are evicted (try_preempt_for, :264-311; truncate_sequence,
     :313-344): a victim keeps at least one block, is cut back to its block boundary (into the
     prompt: re-prefill from there, generated tokens dropped) and goes to the head of the queue;
  2. batch rows (build_batch_rows, :378-505): first one decode row per prefill-complete running
     sequence (token = last generated, or the prompt's last token, at position
     prompt + generated - 1), then prefill rows of the running sequences in order under an
     adaptive token budget (512 / 1024 / 4096 by decode pressure >= 50 % / between / < 25 % of
     max_batch, moving one level per step), rows capped at max_batch. Blocks grow lazily
     (ensure_blocks_for, :346-374);
  3. the model runs every row (writing their KV at their positions); the decode rows' logits give
     one greedy token each (execute_batch, :516-650);
  4. sequences that reached max_gen_len retire and free their blocks (update_sequences, :652-690).

A prompt is never sampled at the end of its prefill: its last token is re-run as the first decode
row, which produces the first generated token (the same tokens as a single-sequence decode that
feeds prompt[:-1] without logits and samples after prompt[-1]).

Deliberate deviation: a sequence that already holds a row of the step being built is never a
preemption victim. The reference excludes only the requester (try_preempt_for, :264-290), so
growing one sequence's blocks can evict another whose row is already in `rows`; that row then
points at freed blocks (-1 in its table) and at a Sequence moved to the waiting queue.
Second deviation: the sequence being admitted leaves the waiting queue before victims are pushed
to its head. The reference holds a reference to the queue's front, pushes the victims in front
of it and then pops the front (try_admit_sequences, :178-253), which drops a victim and leaves
the admitted sequence queued (it would be admitted twice).
Third deviation: a victim cut back into its prompt resumes its prefill at min(its prefill
progress, the cut). The reference resumes at the cut (truncate_sequence, :320-327), which skips
prompt positions never written when the prefill had not reached the cut.

Prefix cache (prefix_cache.cpp, admission at scheduler.cpp:200-246, recording at :483-487): a
fresh request whose prompt starts with whole blocks another sequence has already prefilled mounts
those physical blocks read-only at the front of its block table (reference counts keep them alive)
and starts its prefill after them. Blocks are recorded when the owner's prefill completes; a
lookup takes an entry only while its block is still referenced and still mounted at the recorded
(row, index), so freed, recycled or truncated blocks are never shared.
Deliberate deviations in the prefix cache:
  - the key of block b is the whole token prefix [0, (b + 1) * block_size), compared exactly. The
    reference keys each block by a 64-bit FNV-1a hash of that block's tokens alone, so block b can
    match a block recorded after a different prefix, whose KV (a function of every earlier token)
    differs; and it accepts hash collisions as matches;
  - at most (prompt - 1) // block_size blocks are shared, and an owner records only that many,
    so the block holding a prompt's last position is private on both sides: this scheduler
    re-runs that token as the first decode row, and its KV write must not land in a block other
    sequences read;
  - an entry also records which allocation of the block it saw (a per-block counter bumped on
    every allocation). The reference checks only that the block is referenced and mounted at the
    recorded (row, index); after the owner finishes, the LIFO free list readily gives the same
    block to a new sequence in the same row at the same index, and that block, holding the new
    sequence's KV, would pass both checks.
Sentence-end tokens (update_sequences, :681-690): a sequence whose last generated token is one of
`stop_tokens` retires (the reference asks the model's tokenizer, is_sentence_ending).

Serving timestamps as the reference records them (sequence.h; scheduler.cpp:94, 187, 236, 263,
507, 600-607, 641-647, 662-684), in seconds of time.perf_counter(): arrival_time at add_request,
admit_time at each admission (a resumed sequence is re-stamped), first_token_time when a token
lands on a sequence with none (again after a truncation that dropped them), last_token_time and
the inter-token gaps token_timestamps_ms, finish_time at retirement. batch_reconstruct_times_ms
holds, per decode-only step, the host time spent forming the rows and block tables (the
reference times its pure-decode tensor setup, scheduler.cpp:560-572).
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Callable, Dict, Iterable, List, Optional, Tuple

WAITING, RUNNING, PREEMPTED, FINISHED = "waiting", "running", "preempted", "finished"


class BlockAllocator:
    """Paged KV block pool (block_allocator.cpp): a LIFO free list initialised so blocks are
    handed out 0, 1, 2, ...; per-block reference counts; one block-table row per running
    sequence (rows x max_blocks_per_seq, -1 = empty)."""

    def __init__(self, num_blocks: int, num_rows: int, max_blocks_per_seq: int, block_size: int):
        if num_blocks <= 0 or block_size <= 0:
            raise ValueError("num_blocks and block_size must be positive")
        self.num_blocks, self.num_rows = num_blocks, num_rows
        self.max_blocks_per_seq, self.block_size = max_blocks_per_seq, block_size
        self.free: List[int] = list(range(num_blocks - 1, -1, -1))
        self.ref = [0] * num_blocks
        self.tables = [[-1] * max_blocks_per_seq for _ in range(num_rows)]
        self.row_used = [False] * num_rows  # a row may hold no blocks yet (allocate_blocks(0))
        self.gen = [0] * num_blocks  # bumped on every allocation of a block

    def free_block_count(self) -> int:
        return len(self.free)

    def num_used_blocks(self, row: int) -> int:
        if row < 0 or row >= self.num_rows:
            return 0
        return sum(1 for b in self.tables[row] if b >= 0)

    def _take(self) -> int:
        b = self.free.pop()
        assert self.ref[b] == 0, f"block {b} in the free list with refcount {self.ref[b]}"
        self.ref[b] = 1
        self.gen[b] += 1
        return b

    def allocate_blocks(self, n: int) -> int:
        """A free table row with n fresh blocks; -1 when rows or blocks run out."""
        if n > self.max_blocks_per_seq or n < 0 or len(self.free) < n:
            return -1
        row = next((r for r in range(self.num_rows) if not self.row_used[r]), -1)
        if row < 0:
            return -1
        self.row_used[row] = True
        for i in range(n):
            self.tables[row][i] = self._take()
        return row

    def reserve_shared_prefix(self, row: int, blocks: List[int]) -> bool:
        """Mount `blocks` (already referenced elsewhere) at the front of `row`'s table, shifting
        its own blocks right, and take a reference on each (block_allocator.cpp)."""
        if row < 0 or row >= self.num_rows or not self.row_used[row]:
            return False
        used = self.num_used_blocks(row)
        if used + len(blocks) > self.max_blocks_per_seq:
            return False
        own = self.tables[row][:used]
        self.tables[row][:len(blocks) + used] = list(blocks) + own
        for b in blocks:
            assert self.ref[b] > 0, f"sharing block {b} with refcount 0"
            self.ref[b] += 1
        return True

    def append_blocks(self, row: int, n: int) -> int:
        """Grow a row by n blocks; returns the new block count or -1."""
        if row < 0 or row >= self.num_rows or n <= 0:
            return -1
        used = self.num_used_blocks(row)
        if used + n > self.max_blocks_per_seq or len(self.free) < n:
            return -1
        for i in range(n):
            self.tables[row][used + i] = self._take()
        return used + n

    def free_blocks_from(self, row: int, start: int) -> None:
        if row < 0 or row >= self.num_rows:
            return
        for i in range(start, self.max_blocks_per_seq):
            b = self.tables[row][i]
            if b < 0:
                continue
            self.tables[row][i] = -1
            assert self.ref[b] > 0, f"freeing block {b} with refcount 0"
            self.ref[b] -= 1
            if self.ref[b] == 0:
                self.free.append(b)

    def free_all(self, row: int) -> None:
        self.free_blocks_from(row, 0)
        if 0 <= row < self.num_rows:
            self.row_used[row] = False

    def table_row(self, row: int) -> List[int]:
        return list(self.tables[row])


class PrefixCache:
    """Whole-block prompt prefixes whose KV is committed, for read-only sharing
    (prefix_cache.cpp). Block b of a prompt is keyed by the prompt's tokens [0, (b + 1) *
    block_size) (exact comparison); an entry names the (row, index, block, allocation) that held
    it, and is valid only while that allocation of the block is alive and still mounted there."""

    MAX_ENTRIES = 1 << 16  # a full flush beats unbounded growth (prefix_cache.cpp:47-53)

    def __init__(self, block_size: int):
        self.bs = block_size
        self.map: Dict[Tuple[int, ...], List[Tuple[int, int, int, int]]] = {}

    def lookup(self, prompt: List[int], alloc: BlockAllocator, max_blocks: int) -> List[int]:
        """Physical blocks of the longest shareable whole-block prefix (at most max_blocks)."""
        shared: List[int] = []
        for b in range(min(len(prompt) // self.bs, max_blocks)):
            found = -1
            for row, idx, blk, gen in self.map.get(tuple(prompt[:(b + 1) * self.bs]), ()):
                if alloc.ref[blk] > 0 and alloc.gen[blk] == gen and alloc.tables[row][idx] == blk:
                    found = blk
                    break
            if found < 0:
                break
            shared.append(found)
        return shared

    def insert(self, prompt: List[int], alloc: BlockAllocator, row: int) -> None:
        """Record the prompt blocks of `row` before the one holding the prompt's last position
        (call when its prefill completes): the owner re-runs that position as its first decode
        row, so that block is written again and must stay private."""
        full = (len(prompt) - 1) // self.bs
        if full <= 0:
            return
        if len(self.map) >= self.MAX_ENTRIES:
            self.map.clear()
        for b in range(full):
            entries = self.map.setdefault(tuple(prompt[:(b + 1) * self.bs]), [])
            blk = alloc.tables[row][b]
            entry = (row, b, blk, alloc.gen[blk])
            if entry not in entries:
                entries.append(entry)

    def __len__(self) -> int:
        return len(self.map)


@dataclass
class Sequence:
    id: int
    prompt_tokens: List[int]
    max_gen_len: int
    generated_tokens: List[int] = field(default_factory=list)
    state: str = WAITING
    kv_row: int = -1
    num_blocks: int = 0
    next_prefill: int = 0
    prefill_complete: bool = False
    finished: bool = False
    shared_blocks: int = 0  # prompt blocks mounted from the prefix cache at admission
    arrival_time: float = 0.0
    admit_time: float = 0.0
    first_token_time: float = 0.0
    last_token_time: float = 0.0
    finish_time: float = 0.0
    token_timestamps_ms: List[float] = field(default_factory=list)  # inter-token gaps

    @property
    def num_prompt(self) -> int:
        return len(self.prompt_tokens)


@dataclass
class BatchRow:
    seq: Sequence
    is_decode: bool
    token: int
    position: int


# forward(rows, block tables) -> greedy token of each decode row (decode rows come first)
Forward = Callable[[List[BatchRow], List[List[int]]], List[int]]


class Scheduler:
    def __init__(self, forward: Forward, max_batch: int, max_seq_len: int,
                 max_gen_len: int = 0, block_size: int = 16, num_blocks: Optional[int] = None,
                 prefix_cache: bool = False, stop_tokens: Iterable[int] = ()):
        self.forward = forward
        self.max_batch, self.max_seq_len = max_batch, max_seq_len
        self.max_gen_len = max_gen_len if max_gen_len > 0 else max_seq_len
        self.block_size = block_size
        self.max_blocks_per_seq = (max_seq_len + block_size - 1) // block_size
        if num_blocks is None:  # kv_manager.cpp: the pool covers max_batch full-length sequences
            num_blocks = max_batch * self.max_blocks_per_seq
        self.alloc = BlockAllocator(num_blocks, max_batch, self.max_blocks_per_seq, block_size)
        self.waiting: List[Sequence] = []
        self.running: List[Sequence] = []
        self.finished: List[Sequence] = []
        self.prefill_budget = 1024
        self.next_id = 0
        self.steps = 0
        self.rows_run = 0
        self.preemptions = 0
        self.prefix = PrefixCache(block_size) if prefix_cache else None
        self.stop_tokens = frozenset(int(t) for t in stop_tokens)
        self.shared_prefix_blocks = 0  # blocks mounted from the prefix cache, over the run
        self.batch_reconstruct_times_ms: List[float] = []  # per decode-only step

    @staticmethod
    def resolve_block_size(avg_prompt_len: float) -> int:
        """Block size from the workload's mean prompt length (scheduler.cpp:11-15)."""
        if avg_prompt_len < 64:
            return 8
        if avg_prompt_len > 1024:
            return 32
        return 16

    def add_request(self, prompt: List[int]) -> int:
        """Queue a prompt; -1 when it leaves no room to generate (scheduler.cpp:88-121)."""
        if not prompt or len(prompt) >= self.max_seq_len:
            return -1
        seq = Sequence(self.next_id, list(prompt),
                       max(1, min(self.max_gen_len, self.max_seq_len - len(prompt))))
        seq.arrival_time = time.perf_counter()
        self.next_id += 1
        self.waiting.append(seq)
        return seq.id

    def all_finished(self) -> bool:
        return not self.waiting and not self.running

    def kv_snapshot(self) -> Tuple[int, int, int]:
        """(busy KV rows, tokens held by the running sequences, tokens of KV allocated to them):
        the occupancy the reference's offline benchmark samples before every step
        (benchmark/offline_batch_benchmark.cpp:246-266; get_allocated_kv_tokens,
        scheduler.cpp:700-715)."""
        used = sum(q.num_prompt + len(q.generated_tokens) for q in self.running)
        alloc = sum(q.num_blocks for q in self.running) * self.block_size
        return len(self.running), used, alloc

    # ------------------------------------------------------------------ admission, preemption
    def _admit(self) -> None:
        while self.waiting and len(self.running) < self.max_batch:
            seq = self.waiting[0]
            if seq.state == PREEMPTED:
                self.waiting.pop(0)
                seq.state = RUNNING
                seq.admit_time = time.perf_counter()
                self.running.append(seq)
                continue
            need = (seq.num_prompt + self.block_size - 1) // self.block_size
            self.waiting.pop(0)  # out of the queue before victims are pushed to its head
            shared = self._lookup(seq)
            row = self.alloc.allocate_blocks(need - len(shared))
            if row < 0 and self._preempt_for(need - len(shared), seq.id):
                # eviction may have released the matched blocks: match again
                shared = self._lookup(seq)
                row = self.alloc.allocate_blocks(need - len(shared))
            if row < 0:
                self.waiting.insert(0, seq)  # keeps its place: first in line
                break
            if shared:
                assert self.alloc.reserve_shared_prefix(row, shared)
                seq.next_prefill = len(shared) * self.block_size
                seq.shared_blocks = len(shared)
                self.shared_prefix_blocks += len(shared)
            seq.kv_row, seq.num_blocks, seq.state = row, need, RUNNING
            seq.admit_time = time.perf_counter()
            self.running.append(seq)

    def _lookup(self, seq: Sequence) -> List[int]:
        if self.prefix is None:
            return []
        # the block of the prompt's last position stays private (it is written again)
        return self.prefix.lookup(seq.prompt_tokens, self.alloc,
                                  (seq.num_prompt - 1) // self.block_size)

    def _preempt_for(self, need_blocks: int, skip_id: int, protect=frozenset()) -> bool:
        needed = need_blocks - self.alloc.free_block_count()
        if needed <= 0:
            return True
        victims = []
        for s in reversed(self.running):
            if needed <= 0:
                break
            if s.id == skip_id or s.id in protect or s.state != RUNNING:
                continue
            evictable = s.num_blocks - 1
            if evictable <= 0:
                continue
            take = min(evictable, needed)
            needed -= take
            victims.append((s, take))
        if needed > 0:
            return False
        for s, take in victims:
            self._truncate(s, s.num_blocks - take)
        pre = [s for s in self.running if s.state == PREEMPTED]
        self.running = [s for s in self.running if s.state != PREEMPTED]
        # each preempted sequence is pushed to the front in running order (deque push_front)
        for s in pre:
            self.waiting.insert(0, s)
        return True

    def _truncate(self, seq: Sequence, keep_blocks: int) -> None:
        trunc = keep_blocks * self.block_size
        self.alloc.free_blocks_from(seq.kv_row, keep_blocks)
        seq.num_blocks = keep_blocks
        if trunc < seq.num_prompt:
            # Resume the prefill at the cut, or earlier if it had not got that far yet.
            seq.next_prefill = min(seq.next_prefill, trunc)
            seq.prefill_complete = False
            seq.generated_tokens.clear()
        else:
            keep_gen = trunc - seq.num_prompt
            del seq.generated_tokens[keep_gen:]
        seq.state = PREEMPTED
        self.preemptions += 1

    def _ensure_blocks(self, seq: Sequence, position: int, protect=frozenset()) -> bool:
        needed = position // self.block_size + 1
        if needed > self.max_blocks_per_seq:
            return False
        while seq.num_blocks < needed:
            grown = self.alloc.append_blocks(seq.kv_row, 1)
            if grown <= seq.num_blocks:
                if not self._preempt_for(needed - seq.num_blocks, seq.id, protect):
                    return False
                continue
            seq.num_blocks = grown
        return True

    # ------------------------------------------------------------------ batch formation
    def build_rows(self) -> List[BatchRow]:
        rows: List[BatchRow] = []
        for s in self.running:
            if s.state != RUNNING or s.finished or not s.prefill_complete:
                continue
            if len(rows) >= self.max_batch:
                break
            pos = s.num_prompt + len(s.generated_tokens) - 1
            if not self._ensure_blocks(s, pos, {r.seq.id for r in rows}):
                s.finished, s.state = True, FINISHED
                continue
            tok = s.generated_tokens[-1] if s.generated_tokens else s.prompt_tokens[-1]
            rows.append(BatchRow(s, True, tok, pos))

        if any(s.state == RUNNING and not s.finished and not s.prefill_complete
               for s in self.running):
            backlog = sum(1 for s in self.running if not s.finished and s.prefill_complete)
            pressure = backlog / self.max_batch if self.max_batch > 0 else 0.0
            target = 512 if pressure >= 0.5 else (4096 if pressure < 0.25 else 1024)
            if target > self.prefill_budget:
                self.prefill_budget = min(target, self.prefill_budget * 2)
            elif target < self.prefill_budget:
                self.prefill_budget = max(target, self.prefill_budget // 2)
            self.prefill_budget = max(512, min(4096, self.prefill_budget))
            taken = 0
            for s in self.running:
                if s.state != RUNNING or s.finished or s.prefill_complete:
                    continue
                if taken >= self.prefill_budget or len(rows) >= self.max_batch:
                    break
                take = min(s.num_prompt - s.next_prefill, self.prefill_budget - taken,
                           self.max_batch - len(rows))
                if take <= 0:
                    break
                if not self._ensure_blocks(s, s.next_prefill + take - 1,
                                           {r.seq.id for r in rows}):
                    take = s.num_blocks * self.block_size - s.next_prefill
                    if take <= 0:
                        s.finished, s.state = True, FINISHED
                        continue
                for i in range(take):
                    p = s.next_prefill + i
                    rows.append(BatchRow(s, False, s.prompt_tokens[p], p))
                taken += take
                s.next_prefill += take
                if s.next_prefill >= s.num_prompt:
                    s.prefill_complete = True
                    if self.prefix is not None:  # the prompt's KV is written in this step
                        self.prefix.insert(s.prompt_tokens, self.alloc, s.kv_row)
        return rows

    # ------------------------------------------------------------------ one step
    def step(self) -> None:
        self._admit()
        t0 = time.perf_counter()
        rows = self.build_rows()
        if rows:
            tables = [self.alloc.table_row(r.seq.kv_row) for r in rows]
            nd = sum(1 for r in rows if r.is_decode)
            if nd == len(rows):
                self.batch_reconstruct_times_ms.append((time.perf_counter() - t0) * 1e3)
            tokens = self.forward(rows, tables)
            assert len(tokens) == nd
            now = time.perf_counter()
            for r, t in zip(rows[:nd], tokens):
                q = r.seq
                if not q.generated_tokens:
                    q.first_token_time = now
                else:
                    q.token_timestamps_ms.append((now - q.last_token_time) * 1e3)
                q.last_token_time = now
                q.generated_tokens.append(int(t))
            self.rows_run += len(rows)
        self.steps += 1
        self._retire()

    def _retire(self) -> None:
        keep = []
        for s in self.running:
            stop = (s.prefill_complete and s.generated_tokens and
                    s.generated_tokens[-1] in self.stop_tokens)
            if s.finished or stop or len(s.generated_tokens) >= s.max_gen_len:
                s.finished, s.state = True, FINISHED
                s.finish_time = time.perf_counter()
                self.alloc.free_all(s.kv_row)
                self.finished.append(s)
            else:
                keep.append(s)
        self.running = keep

    def run(self, max_steps: Optional[int] = None) -> List[Sequence]:
        """Step until every request finished. With a pool too small for the running set, eviction
        and resumption can cycle without progress; max_steps bounds that (RuntimeError)."""
        while not self.all_finished():
            if max_steps is not None and self.steps >= max_steps:
                raise RuntimeError(f"scheduler made no progress within {max_steps} steps")
            self.step()
        return sorted(self.finished, key=lambda s: s.id)
