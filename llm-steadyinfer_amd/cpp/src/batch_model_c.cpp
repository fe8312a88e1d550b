// C interface to model::PagedBatchModel and model::Int8Decoder (model/batch_model_c.h).
#include "model/batch_model_c.h"

#include <algorithm>
#include <memory>
#include <string>

#include "model/device_weights.h"
#include "model/int8_decoder.h"
#include "model/paged_batch_model.h"

namespace {

struct Handle {
  std::unique_ptr<model::DeviceWeights> weights;  // when created from a file (outlives model)
  std::unique_ptr<model::PagedBatchModel> model;
  std::string error;
};

Handle* get(void* h) { return static_cast<Handle*>(h); }

int report(Handle* h, const base::Status& st) {
  if (st) return 0;
  h->error = st.get_err_msg();
  return 1;
}

bool fill(const sq8_model_config* cfg, const int8_t* const* qkv_q, const float* const* qkv_s,
          const int8_t* const* o_q, const float* const* o_s, const int8_t* const* gu_q,
          const float* const* gu_s, const int8_t* const* down_q, const float* const* down_s,
          const int8_t* cls_q, const float* cls_s, const float* embedding,
          const float* const* norm, model::BatchModelConfig* c, model::BatchModelWeights* w) {
  if (!cfg || !qkv_q || !qkv_s || !o_q || !o_s || !gu_q || !gu_s || !down_q || !down_s ||
      !norm || cfg->layer_num <= 0)
    return false;
  c->dim = cfg->dim;
  c->hidden_dim = cfg->hidden_dim;
  c->layer_num = cfg->layer_num;
  c->head_num = cfg->head_num;
  c->kv_head_num = cfg->kv_head_num;
  c->vocab_size = cfg->vocab_size;
  c->rope_theta = cfg->rope_theta;
  c->group_size = cfg->group_size;
  c->eps = cfg->eps;
  for (int l = 0; l < c->layer_num; ++l) {
    w->qkv.push_back({qkv_q[l], qkv_s[l]});
    w->o.push_back({o_q[l], o_s[l]});
    w->gu.push_back({gu_q[l], gu_s[l]});
    w->down.push_back({down_q[l], down_s[l]});
  }
  for (int i = 0; i < 2 * c->layer_num + 1; ++i) w->norm.push_back(norm[i]);
  w->cls = {cls_q, cls_s};
  w->embedding = embedding;
  return true;
}

const char* keep_message(const std::string& m) {
  static thread_local std::string msg;
  msg = m;
  return msg.c_str();
}

struct DecoderHandle {
  std::unique_ptr<model::DeviceWeights> weights;  // when created from a file (outlives dec)
  std::unique_ptr<model::Int8Decoder> dec;
  std::string error;
};

// Reads and uploads a model file; nullptr with *error set on failure.
std::unique_ptr<model::DeviceWeights> load(const char* path, bool packed, const char** error) {
  if (!path) {
    if (error) *error = "null path";
    return nullptr;
  }
  model::Int8ModelFile file;
  base::Status st = file.open(path);
  auto w = std::make_unique<model::DeviceWeights>();
  if (st) st = w->upload(file, packed);
  if (!st) {
    if (error) *error = keep_message(st.get_err_msg());
    return nullptr;
  }
  return w;
}

}  // namespace

extern "C" {

void* sq8_decoder_create(const sq8_model_config* cfg, const int8_t* const* qkv_q,
                         const float* const* qkv_s, const int8_t* const* o_q,
                         const float* const* o_s, const int8_t* const* gu_q,
                         const float* const* gu_s, const int8_t* const* down_q,
                         const float* const* down_s, const int8_t* cls_q, const float* cls_s,
                         const float* embedding, const float* const* norm, int max_seq,
                         int split_attention, void* hip_stream, const char** error) {
  model::BatchModelConfig c;
  model::BatchModelWeights w;
  if (!fill(cfg, qkv_q, qkv_s, o_q, o_s, gu_q, gu_s, down_q, down_s, cls_q, cls_s, embedding,
            norm, &c, &w)) {
    if (error) *error = "null argument or no layers";
    return nullptr;
  }
  auto h = std::make_unique<DecoderHandle>();
  h->dec = std::make_unique<model::Int8Decoder>(c, w, max_seq,
                                                static_cast<hipStream_t>(hip_stream),
                                                split_attention != 0);
  const base::Status st = h->dec->init();
  if (!st) {
    if (error) *error = keep_message(st.get_err_msg());
    return nullptr;
  }
  return h.release();
}

void* sq8_decoder_create_from_file(const char* path, int max_seq, int split_attention,
                                   const char** error) {
  auto h = std::make_unique<DecoderHandle>();
  h->weights = load(path, false, error);
  if (!h->weights) return nullptr;
  model::BatchModelConfig c = h->weights->config();
  h->dec = std::make_unique<model::Int8Decoder>(c, h->weights->weights(), max_seq, nullptr,
                                                split_attention != 0);
  const base::Status st = h->dec->init();
  if (!st) {
    if (error) *error = keep_message(st.get_err_msg());
    return nullptr;
  }
  return h.release();
}

void* sq8_batch_model_create_from_file(const char* path, int packed, int max_rows,
                                       int max_seq_len, int num_blocks, int block_size,
                                       int use_graphs, int split_kv, const char** error) {
  auto h = std::make_unique<Handle>();
  h->weights = load(path, packed != 0, error);
  if (!h->weights) return nullptr;
  h->model = std::make_unique<model::PagedBatchModel>(
      h->weights->config(), h->weights->weights(), max_rows, max_seq_len, num_blocks, block_size,
      nullptr, use_graphs != 0, split_kv != 0);
  const base::Status st = h->model->init();
  if (!st) {
    if (error) *error = keep_message(st.get_err_msg());
    return nullptr;
  }
  return h.release();
}

void sq8_decoder_destroy(void* decoder) { delete static_cast<DecoderHandle*>(decoder); }

int sq8_decoder_generate(void* decoder, const int32_t* prompt, int n_prompt, int n_new,
                         int32_t* out, int use_graph) {
  if (!decoder || !prompt || n_prompt <= 0 || n_new < 0 || (n_new > 0 && !out)) return 1;
  auto* h = static_cast<DecoderHandle*>(decoder);
  std::vector<int32_t> toks;
  const base::Status st = h->dec->generate(std::vector<int32_t>(prompt, prompt + n_prompt),
                                           n_new, &toks, use_graph != 0);
  if (!st) {
    h->error = st.get_err_msg();
    return 1;
  }
  std::copy(toks.begin(), toks.end(), out);
  return 0;
}

const char* sq8_decoder_last_error(void* decoder) {
  return decoder ? static_cast<DecoderHandle*>(decoder)->error.c_str() : "null decoder";
}

void* sq8_batch_model_create(const sq8_model_config* cfg, const int8_t* const* qkv_q,
                             const float* const* qkv_s, const int8_t* const* o_q,
                             const float* const* o_s, const int8_t* const* gu_q,
                             const float* const* gu_s, const int8_t* const* down_q,
                             const float* const* down_s, const int8_t* cls_q,
                             const float* cls_s, const float* embedding,
                             const float* const* norm, int packed, int max_rows, int max_seq_len,
                             int num_blocks, int block_size, int use_graphs, int split_kv,
                             void* hip_stream, const char** error) {
  model::BatchModelConfig c;
  model::BatchModelWeights w;
  if (!fill(cfg, qkv_q, qkv_s, o_q, o_s, gu_q, gu_s, down_q, down_s, cls_q, cls_s, embedding,
            norm, &c, &w)) {
    if (error) *error = "null argument or no layers";
    return nullptr;
  }
  w.packed = packed != 0;
  auto h = std::make_unique<Handle>();
  h->model = std::make_unique<model::PagedBatchModel>(
      c, w, max_rows, max_seq_len, num_blocks, block_size, static_cast<hipStream_t>(hip_stream),
      use_graphs != 0, split_kv != 0);
  const base::Status st = h->model->init();
  if (!st) {
    if (error) *error = keep_message(st.get_err_msg());
    return nullptr;
  }
  return h.release();
}

void sq8_batch_model_destroy(void* model) { delete get(model); }

int sq8_batch_model_forward(void* model, int batch, int num_decode_rows, const int32_t* tokens,
                            const int32_t* positions, const int32_t* seq_ids,
                            const int32_t* block_table, int table_stride, int32_t* next_tokens) {
  if (!model || !tokens || !positions || !block_table || (num_decode_rows > 0 && !next_tokens))
    return 1;
  Handle* h = get(model);
  return report(h, h->model->forward_batch(batch, num_decode_rows, tokens, positions, seq_ids,
                                           block_table, table_stride, next_tokens));
}

int sq8_batch_model_capture_decode_graphs(void* model) {
  if (!model) return 1;
  Handle* h = get(model);
  return report(h, h->model->capture_decode_graphs());
}

int sq8_batch_model_stats(void* model, int64_t* out, int n) {
  if (!model || n < 0 || (n > 0 && !out)) return -1;
  const model::PagedBatchModel& m = *get(model)->model;
  const int64_t v[] = {m.graph_replays(), m.rows_run(), static_cast<int64_t>(m.graph_count())};
  const int count = std::min<int>(n, 3);
  std::copy(v, v + count, out);
  return count;
}

const char* sq8_batch_model_last_error(void* model) {
  return model ? get(model)->error.c_str() : "null model";
}

}  // extern "C"
