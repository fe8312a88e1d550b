// Greedy single-sequence INT8 decoder: the reference's single-token forward and generation loop
// (LLamaModel::predict / forward, src/source/model/llama3.cpp:705-818 and :724; Qwen2's
// qwen2.cpp:690-830) on libsq8's fused decode operators (include/sq8_decode.h).
//
// One decode step, 5 launches per layer:
//   QKV GEMV with the residual add + RMSNorm in its prologue (sq8_matmul_rmsnorm; the residual
//   stream ping-pongs between two buffers) -> RoPE + KV write + attention in one launch
//   (sq8_rope_attention_decode[_ws]) -> O GEMV -> gate/up GEMV with add + RMSNorm in its
//   prologue and SwiGLU in its epilogue (sq8_matmul_rmsnorm_swiglu) -> down GEMV;
// then the classifier with the final add + RMSNorm, and one launch for argmax, position advance
// and the next token's embedding (sq8_argmax_advance). Position and token live in device
// memory, so the step is captured once into a HIP graph and replayed per generated token.
// A prompt token runs the same layers without the classifier (embedding first, then
// sq8_step_advance).
//
// The decoder does not own its weights (row-major; the caller keeps them on the device).
#ifndef SQ8_OP_MODEL_INT8_DECODER_H_
#define SQ8_OP_MODEL_INT8_DECODER_H_
#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

#include "base/base.h"
#include "model/paged_batch_model.h"

namespace model {

class Int8Decoder {
 public:
  // stream nullptr: the decoder creates one. split_attention: positions split over several
  // workgroups per head for long contexts (sq8_rope_attention_decode_ws).
  Int8Decoder(const BatchModelConfig& cfg, const BatchModelWeights& weights, int max_seq,
              hipStream_t stream = nullptr, bool split_attention = true);
  ~Int8Decoder();
  Int8Decoder(const Int8Decoder&) = delete;
  Int8Decoder& operator=(const Int8Decoder&) = delete;

  base::Status init();
  // Prompt tokens one step each (no classifier), then n_new greedy tokens; with use_graph each
  // generated token is one replay of the captured step (captured at the first call).
  base::Status generate(const std::vector<int32_t>& prompt, int n_new,
                        std::vector<int32_t>* out, bool use_graph = true);
  hipStream_t stream() const { return stream_; }

 private:
  base::Status launch_step(bool want_logits);
  base::Status check(int rc, const char* what) const;
  base::Status capture();

  BatchModelConfig cfg_;
  BatchModelWeights w_;
  int max_seq_;
  int head_size_ = 0, kv_dim_ = 0;
  bool split_;
  hipStream_t stream_ = nullptr;
  bool owns_stream_ = false;
  bool ready_ = false;
  float *kcache_ = nullptr, *vcache_ = nullptr, *sin_ = nullptr, *cos_ = nullptr;
  float *x_ = nullptr, *x2_ = nullptr, *qkv_ = nullptr, *att_ = nullptr, *proj_ = nullptr,
        *hid_ = nullptr, *logits_ = nullptr;
  int32_t *pos_ = nullptr, *token_ = nullptr, *prompt_d_ = nullptr, *out_d_ = nullptr;
  int prompt_cap_ = 0, out_cap_ = 0;
  int32_t* host_ = nullptr;  // pinned staging of prompts and generated tokens
  int host_cap_ = 0;
  void* ws_ = nullptr;  // matmul workspace (0 bytes for the single-row GEMV shapes)
  size_t ws_bytes_ = 0;
  void* argmax_ws_ = nullptr;
  size_t argmax_ws_bytes_ = 0;
  void* att_ws_ = nullptr;
  size_t att_ws_bytes_ = 0;
  hipGraphExec_t graph_ = nullptr;
};

}  // namespace model
#endif  // SQ8_OP_MODEL_INT8_DECODER_H_
