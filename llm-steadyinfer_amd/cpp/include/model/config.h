// Model configuration of an LLM-SteadyInfer model file. Mirrors the reference's
// src/include/model/config.h:4-33: ModelConfig is the on-disk header (eight int32 and one float,
// 36 bytes, read with one fread), TransformerConfig the values the loader derives from it
// (src/source/model/model.cpp:355-383).
#ifndef SQ8_OP_MODEL_CONFIG_H_
#define SQ8_OP_MODEL_CONFIG_H_
#include <cstdint>

namespace model {

struct ModelConfig {
  int32_t dim = 0;
  int32_t hidden_dim = 0;
  int32_t layer_num = 0;
  int32_t head_num = 0;
  int32_t kv_head_num = 0;
  int32_t vocab_size = 0;  // > 0: classifier shares the embedding; < 0: separate classifier
  int32_t seq_len = 0;
  int32_t immediate_dim_ = 0;
  float rope_theta_ = 1000000.0f;
};
static_assert(sizeof(ModelConfig) == 36, "the header is read with one fread of 36 bytes");

struct TransformerConfig {
  int32_t kv_dim_ = 0;
  int32_t kv_mul_ = 0;
  int32_t head_size_ = 0;
  int32_t vocab_size_ = 0;
  int32_t dim_ = 0;
  int32_t hidden_dim_ = 0;
  int32_t layer_num_ = 0;
  int32_t head_num_ = 0;
  int32_t kv_head_num_ = 0;
  int32_t seq_len_ = 0;
  bool is_shared_weight_ = false;
  int32_t immediate_dim_ = 0;
  float rope_theta_ = 1000000.0f;
};

}  // namespace model
#endif  // SQ8_OP_MODEL_CONFIG_H_
