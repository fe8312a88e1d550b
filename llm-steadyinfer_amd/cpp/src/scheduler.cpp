// Continuous-batching scheduler (src/source/scheduler/scheduler.cpp); the contract and the
// deliberate deviations are in scheduler/scheduler.h.
#include "scheduler/scheduler.h"

#include <algorithm>

namespace scheduler {

namespace {
bool contains(const std::vector<int>& ids, int id) {
  return std::find(ids.begin(), ids.end(), id) != ids.end();
}
}  // namespace

Scheduler::Scheduler(std::shared_ptr<BatchModel> model, int max_batch_size, int max_seq_len,
                     int max_gen_len, int block_size, Options options)
    : model_(std::move(model)),
      max_batch_size_(max_batch_size),
      max_seq_len_(max_seq_len),
      max_gen_len_(max_gen_len > 0 ? max_gen_len : max_seq_len),
      block_size_(block_size > 0 ? block_size : 16) {
  CHECK(model_ != nullptr) << "scheduler without a model";
  CHECK(max_batch_size > 0 && max_seq_len > 0) << "max_batch " << max_batch_size
                                               << ", max_seq_len " << max_seq_len;
  max_blocks_per_seq_ = (max_seq_len_ + block_size_ - 1) / block_size_;
  // The pool covers max_batch full-length sequences unless sized otherwise (kv_manager.cpp).
  const int num_blocks =
      options.num_blocks > 0 ? options.num_blocks : max_batch_size_ * max_blocks_per_seq_;
  alloc_ = std::make_unique<BlockAllocator>(num_blocks, max_batch_size_, max_blocks_per_seq_,
                                            block_size_);
  if (options.prefix_cache) prefix_ = std::make_unique<PrefixCache>(block_size_);
}

int Scheduler::resolve_block_size(long long avg_prompt_len) {
  if (avg_prompt_len < 64) return 8;
  if (avg_prompt_len > 1024) return 32;
  return 16;
}

int Scheduler::add_request(const std::vector<int>& prompt_tokens) {
  const int n = static_cast<int>(prompt_tokens.size());
  if (n == 0 || n >= max_seq_len_) return -1;
  auto seq = std::make_unique<Sequence>();
  seq->id = next_seq_id_++;
  seq->prompt_tokens = prompt_tokens;
  seq->num_prompt_tokens = n;
  seq->max_gen_len = std::max(1, std::min(max_gen_len_, max_seq_len_ - n));
  seq->arrival_time = std::chrono::steady_clock::now();
  Sequence* p = seq.get();
  store_.emplace(p->id, std::move(seq));
  waiting_queue_.push_back(p);
  return p->id;
}

std::vector<const Sequence*> Scheduler::get_running() const {
  return std::vector<const Sequence*>(running_.begin(), running_.end());
}

long long Scheduler::get_allocated_kv_tokens() const {
  long long blocks = 0;
  for (const Sequence* s : running_) blocks += s->num_blocks_allocated;
  return blocks * block_size_;
}

// ---------------------------------------------------------------- admission, preemption
std::vector<int32_t> Scheduler::lookup_prefix(const Sequence& seq) const {
  std::vector<int32_t> shared;
  // The block of the prompt's last position stays private (it is written again).
  if (prefix_) prefix_->lookup(seq.prompt_tokens, *alloc_, &shared,
                               (seq.num_prompt_tokens - 1) / block_size_);
  return shared;
}

void Scheduler::try_admit_sequences() {
  while (!waiting_queue_.empty() && static_cast<int>(running_.size()) < max_batch_size_) {
    Sequence* seq = waiting_queue_.front();
    if (seq->state == SeqState::PREEMPTED) {
      waiting_queue_.pop_front();
      seq->state = SeqState::RUNNING;
      seq->admit_time = std::chrono::steady_clock::now();
      running_.push_back(seq);
      continue;
    }
    const int need = (seq->num_prompt_tokens + block_size_ - 1) / block_size_;
    waiting_queue_.pop_front();  // out of the queue before victims are pushed to its head
    std::vector<int32_t> shared = lookup_prefix(*seq);
    int row = alloc_->allocate_blocks(need - static_cast<int>(shared.size()));
    if (row < 0 && try_preempt_for(need - static_cast<int>(shared.size()), seq->id, {})) {
      shared = lookup_prefix(*seq);  // eviction may have released the matched blocks
      row = alloc_->allocate_blocks(need - static_cast<int>(shared.size()));
    }
    if (row < 0) {
      waiting_queue_.push_front(seq);  // keeps its place: first in line
      break;
    }
    if (!shared.empty()) {
      CHECK(alloc_->reserve_shared_prefix(row, shared)) << "mounting a shared prefix";
      seq->next_prefill_chunk_start = static_cast<int>(shared.size()) * block_size_;
      seq->shared_prefix_blocks = static_cast<int>(shared.size());
      shared_prefix_blocks_ += static_cast<int64_t>(shared.size());
    }
    seq->kv_slot_id = row;
    seq->num_blocks_allocated = need;
    seq->state = SeqState::RUNNING;
    seq->admit_time = std::chrono::steady_clock::now();
    running_.push_back(seq);
  }
}

const Sequence* Scheduler::find_sequence(int id) const {
  for (const Sequence* s : running_)
    if (s->id == id) return s;
  const auto it = store_.find(id);
  if (it != store_.end()) return it->second.get();
  for (const Sequence& s : finished_sequences_)
    if (s.id == id) return &s;
  return nullptr;
}

bool Scheduler::try_preempt_for(int need_blocks, int skip_seq_id,
                                const std::vector<int>& protect) {
  int needed = need_blocks - alloc_->free_block_count();
  if (needed <= 0) return true;
  std::vector<std::pair<Sequence*, int>> victims;
  for (auto it = running_.rbegin(); it != running_.rend() && needed > 0; ++it) {
    Sequence* s = *it;
    if (s->id == skip_seq_id || contains(protect, s->id) || s->state != SeqState::RUNNING)
      continue;
    const int evictable = s->num_blocks_allocated - 1;  // a victim keeps at least one block
    if (evictable <= 0) continue;
    const int take = std::min(evictable, needed);
    needed -= take;
    victims.emplace_back(s, take);
  }
  if (needed > 0) return false;
  for (auto& v : victims) truncate_sequence(*v.first, v.first->num_blocks_allocated - v.second);
  std::vector<Sequence*> keep;
  std::vector<Sequence*> pre;
  for (Sequence* s : running_) (s->state == SeqState::PREEMPTED ? pre : keep).push_back(s);
  running_.swap(keep);
  for (Sequence* s : pre) waiting_queue_.push_front(s);  // each to the head, in running order
  return true;
}

void Scheduler::truncate_sequence(Sequence& seq, int keep_blocks) {
  const int trunc = keep_blocks * block_size_;
  alloc_->free_blocks_from(seq.kv_slot_id, keep_blocks);
  seq.num_blocks_allocated = keep_blocks;
  if (trunc < seq.num_prompt_tokens) {
    // Resume the prefill at the cut, or earlier if it had not got that far yet.
    seq.next_prefill_chunk_start = std::min(seq.next_prefill_chunk_start, trunc);
    seq.is_prefill_complete = false;
    seq.generated_tokens.clear();
  } else {
    const size_t keep_gen = static_cast<size_t>(trunc - seq.num_prompt_tokens);
    if (seq.generated_tokens.size() > keep_gen) seq.generated_tokens.resize(keep_gen);
  }
  seq.num_generated_tokens = static_cast<int>(seq.generated_tokens.size());
  seq.state = SeqState::PREEMPTED;
  ++preemptions_;
}

bool Scheduler::ensure_blocks_for(Sequence* seq, int position, const std::vector<int>& protect) {
  const int needed = position / block_size_ + 1;
  if (needed > max_blocks_per_seq_) return false;
  while (seq->num_blocks_allocated < needed) {
    const int grown = alloc_->append_blocks(seq->kv_slot_id, 1);
    if (grown <= seq->num_blocks_allocated) {
      if (!try_preempt_for(needed - seq->num_blocks_allocated, seq->id, protect)) return false;
      continue;
    }
    seq->num_blocks_allocated = grown;
  }
  return true;
}

// ---------------------------------------------------------------- batch formation
std::vector<Scheduler::BatchRow> Scheduler::build_batch_rows() {
  std::vector<BatchRow> rows;
  std::vector<int> in_rows;  // sequences holding a row of this step: never victims
  // Both passes walk a snapshot: a preemption inside ensure_blocks_for rebuilds running_ without
  // its victims, and a walk by index over the new list would skip the sequence after one. A
  // preempted entry of the snapshot fails the state check.
  const std::vector<Sequence*> snap = running_;
  for (Sequence* s : snap) {
    if (s->state != SeqState::RUNNING || s->is_finished || !s->is_prefill_complete) continue;
    if (static_cast<int>(rows.size()) >= max_batch_size_) break;
    const int pos = s->num_prompt_tokens + static_cast<int>(s->generated_tokens.size()) - 1;
    if (!ensure_blocks_for(s, pos, in_rows)) {
      s->is_finished = true;
      s->state = SeqState::FINISHED;
      continue;
    }
    const int tok = s->generated_tokens.empty() ? s->prompt_tokens.back()
                                                : s->generated_tokens.back();
    rows.push_back(BatchRow{s, true, tok, pos});
    in_rows.push_back(s->id);
  }

  const bool any_prefill = std::any_of(running_.begin(), running_.end(), [](const Sequence* s) {
    return s->state == SeqState::RUNNING && !s->is_finished && !s->is_prefill_complete;
  });
  if (!any_prefill) return rows;

  // Adaptive prefill budget from decode pressure, one level per step.
  const int backlog = static_cast<int>(std::count_if(
      running_.begin(), running_.end(),
      [](const Sequence* s) { return !s->is_finished && s->is_prefill_complete; }));
  const double pressure = static_cast<double>(backlog) / max_batch_size_;
  const int target = pressure >= 0.5 ? 512 : (pressure < 0.25 ? 4096 : 1024);
  if (target > prefill_token_budget_)
    prefill_token_budget_ = std::min(target, prefill_token_budget_ * 2);
  else if (target < prefill_token_budget_)
    prefill_token_budget_ = std::max(target, prefill_token_budget_ / 2);
  prefill_token_budget_ = std::max(512, std::min(4096, prefill_token_budget_));

  int taken = 0;
  const std::vector<Sequence*> snap2 = running_;
  for (Sequence* s : snap2) {
    if (s->state != SeqState::RUNNING || s->is_finished || s->is_prefill_complete) continue;
    if (taken >= prefill_token_budget_ || static_cast<int>(rows.size()) >= max_batch_size_)
      break;
    int take = std::min({s->num_prompt_tokens - s->next_prefill_chunk_start,
                         prefill_token_budget_ - taken,
                         max_batch_size_ - static_cast<int>(rows.size())});
    if (take <= 0) break;
    if (!ensure_blocks_for(s, s->next_prefill_chunk_start + take - 1, in_rows)) {
      take = s->num_blocks_allocated * block_size_ - s->next_prefill_chunk_start;
      if (take <= 0) {
        s->is_finished = true;
        s->state = SeqState::FINISHED;
        continue;
      }
    }
    for (int k = 0; k < take; ++k) {
      const int p = s->next_prefill_chunk_start + k;
      rows.push_back(BatchRow{s, false, s->prompt_tokens[p], p});
    }
    in_rows.push_back(s->id);
    taken += take;
    s->next_prefill_chunk_start += take;
    if (s->next_prefill_chunk_start >= s->num_prompt_tokens) {
      s->is_prefill_complete = true;
      // The prompt's KV is written in this step; later steps may share it.
      if (prefix_) prefix_->insert(s->prompt_tokens, *alloc_, s->kv_slot_id);
    }
  }
  return rows;
}

// ---------------------------------------------------------------- one step
base::Status Scheduler::execute_batch(const std::vector<BatchRow>& rows, TimePoint t0) {
  const int batch = static_cast<int>(rows.size());
  int nd = 0;
  for (const BatchRow& r : rows) nd += r.is_decode;
  tokens_.resize(batch);
  positions_.resize(batch);
  seq_ids_.resize(batch);
  table_.resize(static_cast<size_t>(batch) * max_blocks_per_seq_);
  next_.assign(std::max(nd, 1), 0);
  for (int i = 0; i < batch; ++i) {
    tokens_[i] = rows[i].token_id;
    positions_[i] = rows[i].position;
    seq_ids_[i] = rows[i].seq->id;
    alloc_->copy_block_table_row(rows[i].seq->kv_slot_id,
                                 &table_[static_cast<size_t>(i) * max_blocks_per_seq_]);
  }
  if (nd == batch)
    batch_reconstruct_times_ms_.push_back(
        std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0)
            .count());
  base::Status st = model_->forward_batch(batch, nd, tokens_.data(), positions_.data(),
                                          seq_ids_.data(), table_.data(), max_blocks_per_seq_,
                                          next_.data());
  if (!st) return st;
  const TimePoint now = std::chrono::steady_clock::now();
  for (int i = 0; i < nd; ++i) {
    Sequence* s = rows[i].seq;
    if (s->generated_tokens.empty()) {
      s->first_token_time = now;
    } else {
      s->token_timestamps_ms.push_back(
          std::chrono::duration<double, std::milli>(now - s->last_token_time).count());
    }
    s->last_token_time = now;
    s->generated_tokens.push_back(next_[i]);
    s->num_generated_tokens = static_cast<int>(s->generated_tokens.size());
  }
  rows_run_ += batch;
  return base::error::Success();
}

base::Status Scheduler::step() {
  try_admit_sequences();
  const TimePoint t0 = std::chrono::steady_clock::now();
  const std::vector<BatchRow> rows = build_batch_rows();
  last_rows_.clear();
  for (const BatchRow& r : rows)
    last_rows_.push_back(StepRow{r.seq->id, r.is_decode, r.token_id, r.position});
  base::Status st = base::error::Success();
  if (!rows.empty()) st = execute_batch(rows, t0);
  ++steps_;
  if (!st) {  // unrecoverable forward failure: retire every running sequence
    for (Sequence* s : running_) s->is_finished = true;
  }
  update_sequences();
  return st;
}

void Scheduler::retire(Sequence* s) {
  s->is_finished = true;
  s->state = SeqState::FINISHED;
  s->finish_time = std::chrono::steady_clock::now();
  alloc_->free_all(s->kv_slot_id);
  finished_sequences_.push_back(*s);
  store_.erase(s->id);
}

void Scheduler::update_sequences() {
  std::vector<Sequence*> keep;
  std::vector<Sequence*> done;
  for (Sequence* s : running_) {
    const bool stop = s->is_prefill_complete && !s->generated_tokens.empty() &&
                      model_->is_sentence_ending(s->generated_tokens.back());
    const bool full = static_cast<int>(s->generated_tokens.size()) >= s->max_gen_len;
    (s->is_finished || stop || full ? done : keep).push_back(s);
  }
  running_.swap(keep);
  for (Sequence* s : done) retire(s);
}

base::Status Scheduler::run(int max_steps) {
  while (!all_finished()) {
    if (max_steps > 0 && steps_ >= max_steps)
      return base::error::InternalError("scheduler made no progress within " +
                                        std::to_string(max_steps) + " steps");
    base::Status st = step();
    if (!st) return st;
  }
  return base::error::Success();
}

}  // namespace scheduler
