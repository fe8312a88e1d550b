// One request's host state in the continuous-batching scheduler: the reference's Sequence and
// SeqState (src/include/scheduler/sequence.h), same names and meanings, plus the number of blocks
// mounted from the prefix cache.
#ifndef SQ8_OP_SCHEDULER_SEQUENCE_H_
#define SQ8_OP_SCHEDULER_SEQUENCE_H_
#include <chrono>
#include <vector>

namespace scheduler {

using TimePoint = std::chrono::steady_clock::time_point;

enum class SeqState {
  WAITING,    // queued, no KV blocks yet
  RUNNING,    // admitted, owns a block-table row (may still be prefilling)
  PREEMPTED,  // tail blocks evicted; keeps its row and kept blocks, queued for re-admission
  FINISHED,   // retired: blocks released
};

struct Sequence {
  int id = 0;
  std::vector<int> prompt_tokens;
  std::vector<int> generated_tokens;
  int num_prompt_tokens = 0;
  int num_generated_tokens = 0;
  int kv_slot_id = -1;           // block-table row
  int num_blocks_allocated = 0;  // blocks in the row (shared prefix blocks included)
  SeqState state = SeqState::WAITING;
  bool is_finished = false;
  bool is_prefill_complete = false;
  int next_prefill_chunk_start = 0;  // prompt positions whose KV is written (or shared)
  int max_gen_len = 2048;
  int shared_prefix_blocks = 0;  // prompt blocks mounted from the prefix cache at admission

  // Serving timestamps (scheduler.cpp:94, 187, 236, 263, 507, 600-647, 662-684).
  TimePoint arrival_time;      // add_request
  TimePoint admit_time;        // each admission (a resumed sequence is re-stamped)
  TimePoint first_token_time;  // a token lands on a sequence with none
  TimePoint last_token_time;
  TimePoint finish_time;       // retirement
  std::vector<double> token_timestamps_ms;  // gaps between consecutive generated tokens

  bool is_active() const { return !is_finished; }
  int total_tokens() const { return num_prompt_tokens + num_generated_tokens; }
};

}  // namespace scheduler
#endif  // SQ8_OP_SCHEDULER_SEQUENCE_H_
