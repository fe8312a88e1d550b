/* Plain C interface to scheduler::Scheduler (libsq8_op.so), for hosts that drive it over an FFI
 * (the Python package binds it with ctypes). The model's batched forward is a callback. Every
 * function taking a handle returns a negative value for a NULL handle. No reference counterpart:
 * the reference drives its C++ Scheduler from C++ only (benchmark/, src/source/scheduler). */
#ifndef SQ8_SCHEDULER_C_H_
#define SQ8_SCHEDULER_C_H_
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The batched forward (scheduler::BatchModel::forward_batch): rows 0..batch-1, the first
 * num_decode_rows of them decode rows; block_table is [batch][table_stride]. Writes the greedy
 * token of each decode row to next_tokens; returns 0, or non-zero on failure (the scheduler then
 * retires every running sequence and the step reports SQ8_SCHED_ERR_MODEL). */
typedef int (*sq8_sched_forward_fn)(void* user, int batch, int num_decode_rows,
                                    const int32_t* tokens, const int32_t* positions,
                                    const int32_t* seq_ids, const int32_t* block_table,
                                    int table_stride, int32_t* next_tokens);

enum {
  SQ8_SCHED_OK = 0,
  SQ8_SCHED_ERR_ARG = -1,     /* NULL handle or bad argument */
  SQ8_SCHED_ERR_MODEL = -2,   /* the forward callback failed */
  SQ8_SCHED_ERR_STEPS = -3,   /* run(): max_steps passed before every request finished */
  SQ8_SCHED_ERR_UNKNOWN = -4  /* no such sequence */
};

/* NULL on bad arguments (max_batch, max_seq_len <= 0, block_size or num_blocks < 0, no fn).
 * block_size 0: 16; num_blocks 0: max_batch full-length sequences. */
void* sq8_sched_create(int max_batch, int max_seq_len, int max_gen_len, int block_size,
                       int num_blocks, int prefix_cache, sq8_sched_forward_fn fn, void* user);
void sq8_sched_destroy(void* sched);
/* Token ids that end a sentence (a sequence retires after generating one). */
int sq8_sched_set_stop_tokens(void* sched, const int32_t* tokens, int n);
/* A queued request's id, or -1 (empty prompt, or no room left to generate). */
int sq8_sched_add_request(void* sched, const int32_t* prompt, int n);
int sq8_sched_step(void* sched);
int sq8_sched_run(void* sched, int max_steps);
int sq8_sched_all_finished(void* sched);
/* Counters, as many as fit in n: steps, rows run, preemptions, shared prefix blocks, waiting,
 * running, finished, prefill token budget, free blocks, prefix-cache entries. Returns the count
 * written. */
int sq8_sched_stats(void* sched, int64_t* out, int n);
/* Tokens generated so far by a running or finished sequence (up to cap copied); the count, or
 * SQ8_SCHED_ERR_UNKNOWN. */
int sq8_sched_generated(void* sched, int seq_id, int32_t* out, int cap);
/* Ids of the finished sequences in retirement order (up to cap); the count. */
int sq8_sched_finished_ids(void* sched, int32_t* out, int cap);
/* The last step's rows as (seq id, is_decode, token, position) quadruples (up to cap rows); the
 * row count. */
int sq8_sched_last_rows(void* sched, int32_t* out, int cap);
/* Serving timestamps of a running or finished sequence, in ms since the scheduler was created
 * (-1 when not reached yet): times[0..4] = arrival, admission, first token, last token, finish;
 * its inter-token gaps in ms go to itl (up to cap). Returns the number of gaps, or
 * SQ8_SCHED_ERR_UNKNOWN. */
int sq8_sched_timing(void* sched, int seq_id, double* times, double* itl, int cap);
/* Host ms spent forming each decode-only step's rows (up to cap); returns the count. */
int sq8_sched_batch_reconstruct_times(void* sched, double* out, int cap);
/* KV occupancy now (as the reference's offline benchmark samples it before every step): busy
 * rows, tokens held by the running sequences, tokens of KV allocated to them. Returns the count
 * written (at most n, 3 in all). */
int sq8_sched_kv_snapshot(void* sched, int64_t* out, int n);
/* Reference count of a physical block (0 when free or out of range). */
int sq8_sched_block_ref(void* sched, int block);
/* 1 when the block pool's invariant holds. */
int sq8_sched_invariant(void* sched);

#ifdef __cplusplus
}
#endif
#endif /* SQ8_SCHEDULER_C_H_ */
