// Greedy single-sequence decoder (model/int8_decoder.h) on libsq8's fused decode operators.
#include "model/int8_decoder.h"

#include <algorithm>
#include <cstring>

#include "../../../include/sq8.h"
#include "../../../include/sq8_decode.h"

namespace model {

Int8Decoder::Int8Decoder(const BatchModelConfig& cfg, const BatchModelWeights& weights,
                         int max_seq, hipStream_t stream, bool split_attention)
    : cfg_(cfg), w_(weights), max_seq_(max_seq), split_(split_attention), stream_(stream) {}

Int8Decoder::~Int8Decoder() {
  if (stream_) (void)hipStreamSynchronize(stream_);
  if (graph_) (void)hipGraphExecDestroy(graph_);
  for (void* p : {static_cast<void*>(kcache_), static_cast<void*>(vcache_),
                  static_cast<void*>(sin_), static_cast<void*>(cos_), static_cast<void*>(x_),
                  static_cast<void*>(x2_), static_cast<void*>(qkv_), static_cast<void*>(att_),
                  static_cast<void*>(proj_), static_cast<void*>(hid_),
                  static_cast<void*>(logits_), static_cast<void*>(pos_),
                  static_cast<void*>(token_), static_cast<void*>(prompt_d_),
                  static_cast<void*>(out_d_), ws_, argmax_ws_, att_ws_})
    if (p) (void)hipFree(p);
  if (host_) (void)hipHostFree(host_);
  if (owns_stream_ && stream_) (void)hipStreamDestroy(stream_);
}

base::Status Int8Decoder::check(int rc, const char* what) const {
  if (rc == SQ8_OK) return base::error::Success();
  return base::error::InternalError(std::string(what) + ": " + sq8_status_string(rc));
}

base::Status Int8Decoder::init() {
  const BatchModelConfig& c = cfg_;
  const int L = c.layer_num;
  if (c.dim <= 0 || c.hidden_dim <= 0 || L <= 0 || c.head_num <= 0 || c.kv_head_num <= 0 ||
      c.vocab_size <= 0 || c.group_size <= 0 || c.dim % c.head_num != 0 ||
      c.head_num % c.kv_head_num != 0 || max_seq_ <= 0)
    return base::error::InvalidArgument("model configuration");
  if (w_.packed) return base::error::InvalidArgument("the decoder takes row-major weights");
  const size_t nl = static_cast<size_t>(L);
  if (w_.qkv.size() != nl || w_.o.size() != nl || w_.gu.size() != nl || w_.down.size() != nl ||
      w_.norm.size() != 2 * nl + 1 || !w_.embedding || !w_.cls.q || !w_.cls.s)
    return base::error::InvalidArgument("weights do not match the layer count");
  head_size_ = c.dim / c.head_num;
  kv_dim_ = c.kv_head_num * head_size_;
  if (hipDeviceSynchronize() != hipSuccess) return base::error::InternalError("device");
  if (!stream_) {
    if (hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking) != hipSuccess)
      return base::error::InternalError("stream creation");
    owns_stream_ = true;
  }
  const size_t d = c.dim, kv = kv_dim_, h = c.hidden_dim, S = max_seq_;
  hipError_t e = hipSuccess;
  auto A = [&](void** p, size_t bytes) {
    if (e == hipSuccess) e = hipMalloc(p, std::max<size_t>(bytes, 4));
    if (e == hipSuccess) e = hipMemset(*p, 0, std::max<size_t>(bytes, 4));
  };
  A(reinterpret_cast<void**>(&kcache_), nl * S * kv * 4);
  A(reinterpret_cast<void**>(&vcache_), nl * S * kv * 4);
  A(reinterpret_cast<void**>(&sin_), S * head_size_ * 4);
  A(reinterpret_cast<void**>(&cos_), S * head_size_ * 4);
  A(reinterpret_cast<void**>(&x_), d * 4);
  A(reinterpret_cast<void**>(&x2_), d * 4);
  A(reinterpret_cast<void**>(&qkv_), (d + 2 * kv) * 4);
  A(reinterpret_cast<void**>(&att_), d * 4);
  A(reinterpret_cast<void**>(&proj_), d * 4);
  A(reinterpret_cast<void**>(&hid_), h * 4);
  A(reinterpret_cast<void**>(&logits_), static_cast<size_t>(c.vocab_size) * 4);
  A(reinterpret_cast<void**>(&pos_), 4);
  A(reinterpret_cast<void**>(&token_), 4);
  // Workspaces, zeroed once (their tickets start at zero and every call leaves them so).
  const int gs = c.group_size;
  ws_bytes_ = std::max({sq8_workspace_bytes(1, c.dim + 2 * kv_dim_, c.dim, gs),
                        sq8_workspace_bytes(1, c.dim, c.dim, gs),
                        sq8_workspace_bytes(1, c.dim, c.hidden_dim, gs)});
  if (ws_bytes_) A(&ws_, ws_bytes_);
  argmax_ws_bytes_ = sq8_argmax_workspace_bytes(c.vocab_size);
  if (argmax_ws_bytes_) A(&argmax_ws_, argmax_ws_bytes_);
  if (split_) {
    att_ws_bytes_ = (sq8_decode_attention_workspace_bytes(c.head_num, head_size_, max_seq_) + 3) /
                    4 * 4;
    if (att_ws_bytes_) A(&att_ws_, att_ws_bytes_);
  }
  if (e != hipSuccess) return base::error::InternalError(std::string("allocation: ") +
                                                          hipGetErrorString(e));
  base::Status st = check(sq8_rope_tables(sin_, cos_, head_size_, max_seq_, c.rope_theta,
                                          stream_),
                          "rope tables");
  if (!st) return st;
  if (hipStreamSynchronize(stream_) != hipSuccess) return base::error::InternalError("init");
  ready_ = true;
  return base::error::Success();
}

base::Status Int8Decoder::launch_step(bool want_logits) {
  const BatchModelConfig& c = cfg_;
  const int L = c.layer_num, d = c.dim, kv = kv_dim_, h = c.hidden_dim, gs = c.group_size;
  const size_t layer = static_cast<size_t>(max_seq_) * kv;
  auto mm = [&](const float* x, QuantWeight w, float* y, int N, int K) {
    const bool need = sq8_workspace_bytes(1, N, K, gs) > 0;
    return sq8_matmul(x, w.q, w.s, y, 1, N, K, gs, need ? ws_ : nullptr, need ? ws_bytes_ : 0,
                      stream_);
  };
  int rc = 0;
  float* cur = x_;
  float* other = x2_;
  if (!want_logits) {
    rc = sq8_embedding(w_.embedding, c.vocab_size, d, token_, 1, cur, stream_);
    if (rc) return check(rc, "embedding");
  }
  for (int l = 0; l < L; ++l) {
    if (l == 0) {
      rc = sq8_matmul_rmsnorm(cur, nullptr, nullptr, w_.norm[0], c.eps, w_.qkv[0].q,
                              w_.qkv[0].s, qkv_, d + 2 * kv, d, gs, stream_);
    } else {
      rc = sq8_matmul_rmsnorm(cur, proj_, other, w_.norm[l], c.eps, w_.qkv[l].q, w_.qkv[l].s,
                              qkv_, d + 2 * kv, d, gs, stream_);
      std::swap(cur, other);
    }
    if (rc) return check(rc, "qkv");
    float* kc = kcache_ + l * layer;
    float* vc = vcache_ + l * layer;
    rc = att_ws_ ? sq8_rope_attention_decode_ws(qkv_, c.head_num, c.kv_head_num, head_size_,
                                                pos_, sin_, cos_, kc, vc, att_, max_seq_,
                                                att_ws_, att_ws_bytes_, stream_)
                 : sq8_rope_attention_decode(qkv_, c.head_num, c.kv_head_num, head_size_, pos_,
                                             sin_, cos_, kc, vc, att_, max_seq_, stream_);
    if (rc) return check(rc, "attention");
    rc = mm(att_, w_.o[l], proj_, d, d);
    if (rc) return check(rc, "o");
    rc = sq8_matmul_rmsnorm_swiglu(cur, proj_, other, w_.norm[L + l], c.eps, w_.gu[l].q,
                                   w_.gu[l].s, hid_, 2 * h, d, gs, stream_);
    std::swap(cur, other);
    if (rc) return check(rc, "gate/up");
    rc = mm(hid_, w_.down[l], proj_, d, h);
    if (rc) return check(rc, "down");
  }
  if (want_logits) {
    rc = sq8_matmul_rmsnorm(cur, proj_, nullptr, w_.norm[2 * L], c.eps, w_.cls.q, w_.cls.s,
                            logits_, c.vocab_size, d, gs, stream_);
    if (rc) return check(rc, "classifier");
    // token = argmax, pos += 1, x_ = embedding of the token (the next step starts from x_).
    rc = sq8_argmax_advance(logits_, c.vocab_size, argmax_ws_, argmax_ws_bytes_, pos_, token_,
                            w_.embedding, c.vocab_size, d, x_, stream_);
    if (rc) return check(rc, "argmax");
  } else {
    rc = sq8_step_advance(pos_, token_, token_, stream_);
    if (rc) return check(rc, "advance");
  }
  return base::error::Success();
}

base::Status Int8Decoder::capture() {
  hipGraph_t g = nullptr;
  if (hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal) != hipSuccess)
    return base::error::InternalError("begin capture");
  base::Status st = launch_step(true);
  const hipError_t e = hipStreamEndCapture(stream_, &g);
  if (!st) {
    if (g) (void)hipGraphDestroy(g);
    return st;
  }
  if (e != hipSuccess || !g) return base::error::InternalError("end capture");
  const hipError_t ei = hipGraphInstantiate(&graph_, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  return ei == hipSuccess ? base::error::Success()
                          : base::error::InternalError("graph instantiation");
}

base::Status Int8Decoder::generate(const std::vector<int32_t>& prompt, int n_new,
                                   std::vector<int32_t>* out, bool use_graph) {
  if (!ready_) return base::error::InternalError("init() not called");
  const int np = static_cast<int>(prompt.size());
  if (np == 0 || n_new < 0 || np + n_new > max_seq_)
    return base::error::InvalidArgument("prompt + new tokens must fit max_seq");
  for (int32_t t : prompt)
    if (t < 0 || t >= cfg_.vocab_size) return base::error::InvalidArgument("token id");
  hipError_t e = hipStreamSynchronize(stream_);
  // Staging: the prompt and the generated tokens (device) and one pinned host array.
  auto grow = [&](int32_t** p, int* cap, int n) {
    if (e != hipSuccess || n <= *cap) return;
    if (*p) e = hipFree(*p);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(p), n * sizeof(int32_t));
    if (e == hipSuccess) *cap = n;
  };
  grow(&prompt_d_, &prompt_cap_, np);
  grow(&out_d_, &out_cap_, std::max(n_new, 1));
  if (e == hipSuccess && std::max(np, n_new) > host_cap_) {
    if (host_) e = hipHostFree(host_);
    host_ = nullptr;
    if (e == hipSuccess)
      e = hipHostMalloc(reinterpret_cast<void**>(&host_), std::max(np, n_new) * sizeof(int32_t),
                        hipHostMallocDefault);
    if (e == hipSuccess) host_cap_ = std::max(np, n_new);
  }
  if (e != hipSuccess) return base::error::InternalError("staging");
  std::memcpy(host_, prompt.data(), np * sizeof(int32_t));
  // reset: position 0, empty caches
  e = hipMemcpyAsync(prompt_d_, host_, np * sizeof(int32_t), hipMemcpyHostToDevice, stream_);
  if (e == hipSuccess) e = hipMemsetAsync(pos_, 0, sizeof(int32_t), stream_);
  const size_t cache = static_cast<size_t>(cfg_.layer_num) * max_seq_ * kv_dim_ * sizeof(float);
  if (e == hipSuccess) e = hipMemsetAsync(kcache_, 0, cache, stream_);
  if (e == hipSuccess) e = hipMemsetAsync(vcache_, 0, cache, stream_);
  if (e != hipSuccess) return base::error::InternalError("reset");
  for (int i = 0; i + 1 < np; ++i) {  // prompt tokens: no classifier
    e = hipMemcpyAsync(token_, prompt_d_ + i, sizeof(int32_t), hipMemcpyDeviceToDevice, stream_);
    if (e != hipSuccess) return base::error::InternalError("token");
    base::Status st = launch_step(false);
    if (!st) return st;
  }
  e = hipMemcpyAsync(token_, prompt_d_ + np - 1, sizeof(int32_t), hipMemcpyDeviceToDevice,
                     stream_);
  if (e != hipSuccess) return base::error::InternalError("token");
  if (use_graph && !graph_) {
    base::Status st = capture();
    if (!st) return st;
  }
  // The first decode step starts from the last prompt token's embedding.
  int rc = sq8_embedding(w_.embedding, cfg_.vocab_size, cfg_.dim, token_, 1, x_, stream_);
  if (rc) return check(rc, "embedding");
  for (int i = 0; i < n_new; ++i) {
    if (use_graph) {
      if (hipGraphLaunch(graph_, stream_) != hipSuccess)
        return base::error::InternalError("graph launch");
    } else {
      base::Status st = launch_step(true);
      if (!st) return st;
    }
    e = hipMemcpyAsync(out_d_ + i, token_, sizeof(int32_t), hipMemcpyDeviceToDevice, stream_);
    if (e != hipSuccess) return base::error::InternalError("token copy");
  }
  if (n_new > 0)
    e = hipMemcpyAsync(host_, out_d_, n_new * sizeof(int32_t), hipMemcpyDeviceToHost, stream_);
  if (e == hipSuccess) e = hipStreamSynchronize(stream_);
  if (e != hipSuccess) return base::error::InternalError(std::string("generate: ") +
                                                          hipGetErrorString(e));
  out->assign(host_, host_ + n_new);
  return base::error::Success();
}

}  // namespace model
