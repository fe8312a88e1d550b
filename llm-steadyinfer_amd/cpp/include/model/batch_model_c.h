/* Plain C interface to model::PagedBatchModel and model::Int8Decoder (libsq8_op.so). sq8_batch_model_forward has the
 * signature of sq8_sched_forward_fn (scheduler/scheduler_c.h), so a native scheduler can drive
 * the native model with no host language in between. No reference counterpart: the reference
 * calls its C++ model from C++ only. */
#ifndef SQ8_BATCH_MODEL_C_H_
#define SQ8_BATCH_MODEL_C_H_
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct sq8_model_config {
  int dim, hidden_dim, layer_num, head_num, kv_head_num, vocab_size;
  float rope_theta;
  int group_size;
  float eps;
} sq8_model_config;

/* Device pointers, layer_num of each per-layer array (norm: 2 layer_num + 1: attention norms,
 * FFN norms, final norm). qkv is [wq; wk; wv], gu is [w1; w3]. With packed != 0 the projections
 * are in the sq8_pack_weights layout. The caller keeps the weights alive. hip_stream NULL: the
 * model creates its own stream. Returns NULL on failure, with a message in *error (a static
 * string) when error is not NULL. */
void* sq8_batch_model_create(const sq8_model_config* cfg, const int8_t* const* qkv_q,
                             const float* const* qkv_s, const int8_t* const* o_q,
                             const float* const* o_s, const int8_t* const* gu_q,
                             const float* const* gu_s, const int8_t* const* down_q,
                             const float* const* down_s, const int8_t* cls_q,
                             const float* cls_s, const float* embedding,
                             const float* const* norm, int packed, int max_rows, int max_seq_len,
                             int num_blocks, int block_size, int use_graphs, int split_kv,
                             void* hip_stream, const char** error);
void sq8_batch_model_destroy(void* model);
/* One step (scheduler::BatchModel::forward_batch); 0 or non-zero on failure
 * (sq8_batch_model_last_error says why). */
int sq8_batch_model_forward(void* model, int batch, int num_decode_rows, const int32_t* tokens,
                            const int32_t* positions, const int32_t* seq_ids,
                            const int32_t* block_table, int table_stride, int32_t* next_tokens);
int sq8_batch_model_capture_decode_graphs(void* model);
/* graph replays, rows run, captured graphs (as many as fit in n); returns the count written. */
int sq8_batch_model_stats(void* model, int64_t* out, int n);
const char* sq8_batch_model_last_error(void* model);

/* model::Int8Decoder, the greedy single-sequence decoder (row-major weights, arguments as
 * sq8_batch_model_create). generate: prompt tokens one step each, then n_new greedy tokens into
 * out; use_graph: one HIP-graph replay per generated token. Returns 0, or non-zero with a
 * message in sq8_decoder_last_error. */
void* sq8_decoder_create(const sq8_model_config* cfg, const int8_t* const* qkv_q,
                         const float* const* qkv_s, const int8_t* const* o_q,
                         const float* const* o_s, const int8_t* const* gu_q,
                         const float* const* gu_s, const int8_t* const* down_q,
                         const float* const* down_s, const int8_t* cls_q, const float* cls_s,
                         const float* embedding, const float* const* norm, int max_seq,
                         int split_attention, void* hip_stream, const char** error);
void sq8_decoder_destroy(void* decoder);
int sq8_decoder_generate(void* decoder, const int32_t* prompt, int n_prompt, int n_new,
                         int32_t* out, int use_graph);
const char* sq8_decoder_last_error(void* decoder);

/* The same models from an INT8 model file (the reference's .bin layout), read by the C++ loader
 * (model::Int8ModelFile) and uploaded fused (model::DeviceWeights); the handle owns the device
 * weights. Destroy with sq8_batch_model_destroy / sq8_decoder_destroy. */
void* sq8_batch_model_create_from_file(const char* path, int packed, int max_rows,
                                       int max_seq_len, int num_blocks, int block_size,
                                       int use_graphs, int split_kv, const char** error);
void* sq8_decoder_create_from_file(const char* path, int max_seq, int split_attention,
                                   const char** error);

#ifdef __cplusplus
}
#endif
#endif /* SQ8_BATCH_MODEL_C_H_ */
