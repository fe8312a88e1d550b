// C interface to scheduler::Scheduler (scheduler/scheduler_c.h): the model is a callback.
#include "scheduler/scheduler_c.h"

#include <algorithm>
#include <memory>
#include <unordered_set>
#include <vector>

#include "scheduler/scheduler.h"

namespace {

class CallbackModel : public scheduler::BatchModel {
 public:
  CallbackModel(sq8_sched_forward_fn fn, void* user) : fn_(fn), user_(user) {}
  base::Status forward_batch(int batch, int num_decode_rows, const int32_t* tokens,
                             const int32_t* positions, const int32_t* seq_ids,
                             const int32_t* block_table, int table_stride,
                             int32_t* next_tokens) override {
    const int rc = fn_(user_, batch, num_decode_rows, tokens, positions, seq_ids, block_table,
                       table_stride, next_tokens);
    return rc == 0 ? base::error::Success()
                   : base::error::InternalError("forward callback returned " + std::to_string(rc));
  }
  bool is_sentence_ending(int32_t token) const override { return stop_.count(token) != 0; }
  std::unordered_set<int32_t> stop_;

 private:
  sq8_sched_forward_fn fn_;
  void* user_;
};

struct Handle {
  std::shared_ptr<CallbackModel> model;
  std::unique_ptr<scheduler::Scheduler> sched;
};

Handle* get(void* h) { return static_cast<Handle*>(h); }

const scheduler::Sequence* find_seq(const scheduler::Scheduler& s, int id) {
  for (const scheduler::Sequence* q : s.get_running())
    if (q->id == id) return q;
  for (const scheduler::Sequence& q : s.get_finished())
    if (q.id == id) return &q;
  return nullptr;
}

}  // namespace

extern "C" {

void* sq8_sched_create(int max_batch, int max_seq_len, int max_gen_len, int block_size,
                       int num_blocks, int prefix_cache, sq8_sched_forward_fn fn, void* user) {
  if (max_batch <= 0 || max_seq_len <= 0 || block_size < 0 || num_blocks < 0 || !fn)
    return nullptr;
  auto* h = new Handle;
  h->model = std::make_shared<CallbackModel>(fn, user);
  scheduler::Scheduler::Options opt;
  opt.num_blocks = num_blocks;
  opt.prefix_cache = prefix_cache != 0;
  h->sched = std::make_unique<scheduler::Scheduler>(h->model, max_batch, max_seq_len,
                                                    max_gen_len, block_size, opt);
  return h;
}

void sq8_sched_destroy(void* sched) { delete get(sched); }

int sq8_sched_set_stop_tokens(void* sched, const int32_t* tokens, int n) {
  if (!sched || n < 0 || (n > 0 && !tokens)) return SQ8_SCHED_ERR_ARG;
  get(sched)->model->stop_.clear();
  get(sched)->model->stop_.insert(tokens, tokens + n);
  return SQ8_SCHED_OK;
}

int sq8_sched_add_request(void* sched, const int32_t* prompt, int n) {
  if (!sched || n < 0 || (n > 0 && !prompt)) return SQ8_SCHED_ERR_ARG;
  return get(sched)->sched->add_request(std::vector<int>(prompt, prompt + n));
}

int sq8_sched_step(void* sched) {
  if (!sched) return SQ8_SCHED_ERR_ARG;
  return get(sched)->sched->step() ? SQ8_SCHED_OK : SQ8_SCHED_ERR_MODEL;
}

int sq8_sched_run(void* sched, int max_steps) {
  if (!sched) return SQ8_SCHED_ERR_ARG;
  scheduler::Scheduler& s = *get(sched)->sched;
  while (!s.all_finished()) {
    if (max_steps > 0 && s.steps() >= max_steps) return SQ8_SCHED_ERR_STEPS;
    if (!s.step()) return SQ8_SCHED_ERR_MODEL;
  }
  return SQ8_SCHED_OK;
}

int sq8_sched_all_finished(void* sched) {
  if (!sched) return SQ8_SCHED_ERR_ARG;
  return get(sched)->sched->all_finished() ? 1 : 0;
}

int sq8_sched_stats(void* sched, int64_t* out, int n) {
  if (!sched || n < 0 || (n > 0 && !out)) return SQ8_SCHED_ERR_ARG;
  const scheduler::Scheduler& s = *get(sched)->sched;
  const int64_t v[] = {s.steps(),
                       s.rows_run(),
                       s.preemptions(),
                       s.shared_prefix_blocks(),
                       s.num_waiting(),
                       s.get_busy_kv_slots(),
                       static_cast<int64_t>(s.get_finished().size()),
                       s.prefill_token_budget(),
                       s.block_allocator().free_block_count(),
                       s.prefix_cache() ? static_cast<int64_t>(s.prefix_cache()->entry_count())
                                        : 0};
  const int count = std::min<int>(n, sizeof(v) / sizeof(v[0]));
  std::copy(v, v + count, out);
  return count;
}

int sq8_sched_generated(void* sched, int seq_id, int32_t* out, int cap) {
  if (!sched || cap < 0 || (cap > 0 && !out)) return SQ8_SCHED_ERR_ARG;
  const scheduler::Sequence* q = find_seq(*get(sched)->sched, seq_id);
  if (!q) return SQ8_SCHED_ERR_UNKNOWN;
  const int n = static_cast<int>(q->generated_tokens.size());
  std::copy_n(q->generated_tokens.begin(), std::min(n, cap), out);
  return n;
}

int sq8_sched_finished_ids(void* sched, int32_t* out, int cap) {
  if (!sched || cap < 0 || (cap > 0 && !out)) return SQ8_SCHED_ERR_ARG;
  const auto& f = get(sched)->sched->get_finished();
  const int n = static_cast<int>(f.size());
  for (int i = 0; i < std::min(n, cap); ++i) out[i] = f[i].id;
  return n;
}

int sq8_sched_last_rows(void* sched, int32_t* out, int cap) {
  if (!sched || cap < 0 || (cap > 0 && !out)) return SQ8_SCHED_ERR_ARG;
  const auto& rows = get(sched)->sched->last_rows();
  const int n = static_cast<int>(rows.size());
  for (int i = 0; i < std::min(n, cap); ++i) {
    out[4 * i] = rows[i].seq_id;
    out[4 * i + 1] = rows[i].is_decode ? 1 : 0;
    out[4 * i + 2] = rows[i].token_id;
    out[4 * i + 3] = rows[i].position;
  }
  return n;
}

int sq8_sched_timing(void* sched, int seq_id, double* times, double* itl, int cap) {
  if (!sched || !times || cap < 0 || (cap > 0 && !itl)) return SQ8_SCHED_ERR_ARG;
  const scheduler::Scheduler& s = *get(sched)->sched;
  const scheduler::Sequence* q = s.find_sequence(seq_id);
  if (!q) return SQ8_SCHED_ERR_UNKNOWN;
  const scheduler::TimePoint t0 = s.created();
  auto ms = [&](scheduler::TimePoint t) {
    return t == scheduler::TimePoint{} ? -1.0
                                       : std::chrono::duration<double, std::milli>(t - t0).count();
  };
  times[0] = ms(q->arrival_time);
  times[1] = ms(q->admit_time);
  times[2] = ms(q->first_token_time);
  times[3] = ms(q->last_token_time);
  times[4] = ms(q->finish_time);
  const int n = static_cast<int>(q->token_timestamps_ms.size());
  std::copy_n(q->token_timestamps_ms.begin(), std::min(n, cap), itl);
  return n;
}

int sq8_sched_batch_reconstruct_times(void* sched, double* out, int cap) {
  if (!sched || cap < 0 || (cap > 0 && !out)) return SQ8_SCHED_ERR_ARG;
  const auto& v = get(sched)->sched->get_batch_reconstruct_times_ms();
  const int n = static_cast<int>(v.size());
  std::copy_n(v.begin(), std::min(n, cap), out);
  return n;
}

int sq8_sched_kv_snapshot(void* sched, int64_t* out, int n) {
  if (!sched || n < 0 || (n > 0 && !out)) return SQ8_SCHED_ERR_ARG;
  const scheduler::Scheduler& s = *get(sched)->sched;
  int64_t used = 0;
  for (const scheduler::Sequence* q : s.get_running())
    used += q->num_prompt_tokens + static_cast<int64_t>(q->generated_tokens.size());
  const int64_t v[] = {s.get_busy_kv_slots(), used, s.get_allocated_kv_tokens()};
  const int count = std::min(n, 3);
  std::copy(v, v + count, out);
  return count;
}

int sq8_sched_block_ref(void* sched, int block) {
  if (!sched) return SQ8_SCHED_ERR_ARG;
  return get(sched)->sched->block_allocator().ref_count(block);
}

int sq8_sched_invariant(void* sched) {
  if (!sched) return SQ8_SCHED_ERR_ARG;
  return get(sched)->sched->block_allocator().invariant_holds() ? 1 : 0;
}

}  // extern "C"
