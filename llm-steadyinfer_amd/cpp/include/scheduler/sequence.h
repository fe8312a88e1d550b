// One request's host state in the continuous-batching scheduler: the reference's Sequence and
// SeqState (src/include/scheduler/sequence.h), same names and meanings; the latency timestamps
// are left out and the blocks mounted from the prefix cache are counted.
#ifndef SQ8_OP_SCHEDULER_SEQUENCE_H_
#define SQ8_OP_SCHEDULER_SEQUENCE_H_
#include <vector>

namespace scheduler {

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

  bool is_active() const { return !is_finished; }
  int total_tokens() const { return num_prompt_tokens + num_generated_tokens; }
};

}  // namespace scheduler
#endif  // SQ8_OP_SCHEDULER_SEQUENCE_H_
