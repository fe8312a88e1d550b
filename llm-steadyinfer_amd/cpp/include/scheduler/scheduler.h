// Continuous-batching scheduler over a paged KV block pool: the reference's Scheduler
// (src/include/scheduler/scheduler.h, src/source/scheduler/scheduler.cpp), same public
// interface, driving any BatchModel (the batched forward over the paged cache).
//
// One step (Scheduler::step, scheduler.cpp:122-164):
//  1. admission (try_admit_sequences, :170-262): waiting sequences become RUNNING while fewer
//     than max_batch run. A fresh one gets a block-table row with its prompt's blocks (after any
//     prefix-cache blocks mounted in front); a preempted one resumes with the blocks it kept.
//     When the pool is short, tail blocks of the most recently admitted running sequences are
//     evicted (try_preempt_for, :264-311; truncate_sequence, :313-344): a victim keeps at least
//     one block, is cut back to a block boundary and queued at the head;
//  2. batch rows (build_batch_rows, :378-505): one decode row per prefill-complete sequence
//     (the last generated token, or the prompt's last token, at position prompt + generated - 1),
//     then prefill rows in running order under an adaptive token budget (512 / 1024 / 4096 by
//     decode pressure >= 50 % / between / < 25 % of max_batch, one level per step), at most
//     max_batch rows. Blocks grow lazily (ensure_blocks_for, :346-374);
//  3. the model runs every row (writing their KV at their positions); each decode row yields one
//     greedy token (execute_batch, :516-650);
//  4. sequences at max_gen_len, or whose last token ends a sentence, retire and free their
//     blocks (update_sequences, :652-690).
//
// A prompt is never sampled at the end of its prefill: its last token is re-run as the first
// decode row, which produces the first generated token.
//
// Deliberate deviations (each fixes a reference case that corrupts state):
//  - a sequence that already holds a row of the step being built is never a preemption victim
//    (the reference excludes only the requester, so a row could point at freed blocks);
//  - the sequence being admitted leaves the queue before victims are pushed to its head (the
//    reference pops the front after pushing them, dropping a victim and keeping the admitted
//    sequence queued);
//  - a victim cut back into its prompt resumes its prefill at min(its progress, the cut) (the
//    reference resumes at the cut, skipping positions never written).
// Serving timestamps are kept per Sequence as the reference keeps them, and
// get_batch_reconstruct_times_ms() holds, per decode-only step, the host time spent forming the
// rows and block tables.
#ifndef SQ8_OP_SCHEDULER_SCHEDULER_H_
#define SQ8_OP_SCHEDULER_SCHEDULER_H_
#include <cstdint>
#include <deque>
#include <memory>
#include <unordered_map>
#include <vector>

#include "base/base.h"
#include "scheduler/block_allocator.h"
#include "scheduler/prefix_cache.h"
#include "scheduler/sequence.h"

namespace scheduler {

// The batched forward the scheduler drives (the role of the reference's model::Model
// forward_batch / decode_step / post_processing_batch, scheduler.cpp:516-650).
class BatchModel {
 public:
  virtual ~BatchModel() = default;
  // Rows 0 .. batch-1: token ids, positions, and block tables ([batch][table_stride], -1 =
  // empty); seq_ids names each row's sequence. The first num_decode_rows rows are decode rows
  // (prefill rows follow, those of one sequence in position order). Writes every row's KV at
  // its position, then the greedy token of each decode row to next_tokens[0 .. num_decode_rows).
  virtual base::Status forward_batch(int batch, int num_decode_rows, const int32_t* tokens,
                                     const int32_t* positions, const int32_t* seq_ids,
                                     const int32_t* block_table, int table_stride,
                                     int32_t* next_tokens) = 0;
  // Sentence-end token (model::Model::is_sentence_ending): the sequence retires after it.
  virtual bool is_sentence_ending(int32_t token) const {
    (void)token;
    return false;
  }
};

struct SchedulerOptions {
  int num_blocks = 0;         // 0: max_batch full-length sequences (kv_manager.cpp)
  bool prefix_cache = false;  // the reference enables it unless LLAMA_DISABLE_PREFIX_CACHE=1
};

class Scheduler {
 public:
  using Options = SchedulerOptions;

  // max_seq_len: per-sequence KV capacity (prompt + generation); max_gen_len: per-request
  // generation limit (0: max_seq_len; clamped to the room a prompt leaves); block_size: paged
  // block size (0: 16).
  Scheduler(std::shared_ptr<BatchModel> model, int max_batch_size, int max_seq_len,
            int max_gen_len = 0, int block_size = 0, Options options = Options());

  // Queue a prompt; its id, or -1 when it is empty or leaves no room to generate.
  int add_request(const std::vector<int>& prompt_tokens);
  // One scheduling iteration; an error when the model's forward fails (every running sequence
  // is then retired, as force_finish_all does).
  base::Status step();
  // Step until every request finished; an error if max_steps (> 0) pass first: with a pool too
  // small for the running set, eviction and resumption can cycle without progress.
  base::Status run(int max_steps = 0);
  bool all_finished() const { return waiting_queue_.empty() && running_.empty(); }

  // Finished sequences in retirement order; running ones in admission order.
  const std::vector<Sequence>& get_finished() const { return finished_sequences_; }
  std::vector<const Sequence*> get_running() const;
  int num_waiting() const { return static_cast<int>(waiting_queue_.size()); }
  const std::vector<double>& get_batch_reconstruct_times_ms() const {
    return batch_reconstruct_times_ms_;
  }
  // The running or finished sequence with this id (nullptr if none).
  const Sequence* find_sequence(int id) const;
  TimePoint created() const { return created_; }
  int get_block_size() const { return block_size_; }
  int get_max_kv_seq_len() const { return max_seq_len_; }
  int get_busy_kv_slots() const { return static_cast<int>(running_.size()); }
  long long get_allocated_kv_tokens() const;
  // Block size from the workload's mean prompt length (scheduler.cpp:11-15).
  static int resolve_block_size(long long avg_prompt_len);

  const BlockAllocator& block_allocator() const { return *alloc_; }
  const PrefixCache* prefix_cache() const { return prefix_.get(); }
  int64_t steps() const { return steps_; }
  int64_t rows_run() const { return rows_run_; }
  int64_t preemptions() const { return preemptions_; }
  int64_t shared_prefix_blocks() const { return shared_prefix_blocks_; }
  int prefill_token_budget() const { return prefill_token_budget_; }

  // One row of the last step's batch, as handed to the model.
  struct StepRow {
    int seq_id = -1;
    bool is_decode = false;
    int32_t token_id = 0;
    int32_t position = 0;
  };
  const std::vector<StepRow>& last_rows() const { return last_rows_; }

 private:
  // One row of the batch being built (build_batch_rows).
  struct BatchRow {
    Sequence* seq = nullptr;
    bool is_decode = false;
    int32_t token_id = 0;
    int32_t position = 0;
  };

  void try_admit_sequences();
  std::vector<int32_t> lookup_prefix(const Sequence& seq) const;
  bool try_preempt_for(int need_blocks, int skip_seq_id, const std::vector<int>& protect);
  void truncate_sequence(Sequence& seq, int keep_blocks);
  bool ensure_blocks_for(Sequence* seq, int position, const std::vector<int>& protect);
  std::vector<BatchRow> build_batch_rows();
  base::Status execute_batch(const std::vector<BatchRow>& rows, TimePoint t0);
  void update_sequences();
  void retire(Sequence* seq);

  std::shared_ptr<BatchModel> model_;
  std::unique_ptr<BlockAllocator> alloc_;
  std::unique_ptr<PrefixCache> prefix_;
  std::unordered_map<int, std::unique_ptr<Sequence>> store_;  // owns every live sequence
  std::deque<Sequence*> waiting_queue_;          // preempted sequences jump the head
  std::vector<Sequence*> running_;
  std::vector<Sequence> finished_sequences_;
  std::vector<StepRow> last_rows_;
  std::vector<double> batch_reconstruct_times_ms_;
  TimePoint created_ = std::chrono::steady_clock::now();
  int max_batch_size_;
  int max_seq_len_;
  int max_gen_len_;
  int block_size_;
  int max_blocks_per_seq_;
  int next_seq_id_ = 0;
  int prefill_token_budget_ = 1024;
  int64_t steps_ = 0;
  int64_t rows_run_ = 0;
  int64_t preemptions_ = 0;
  int64_t shared_prefix_blocks_ = 0;
  // Per-step staging of the model's inputs (reused, no allocation once grown).
  std::vector<int32_t> tokens_, positions_, seq_ids_, table_, next_;
};

}  // namespace scheduler
#endif  // SQ8_OP_SCHEDULER_SCHEDULER_H_
