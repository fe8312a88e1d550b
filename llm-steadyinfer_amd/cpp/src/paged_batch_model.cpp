// Batched forward over the paged KV cache (model/paged_batch_model.h): the launch sequence of
// the reference's forward_batch (src/source/model/llama3.cpp:996-1194) on libsq8's C ABI.
#include "model/paged_batch_model.h"

#include <algorithm>
#include <cstring>

#include "../../../include/sq8.h"
#include "../../../include/sq8_batch.h"
#include "../../../include/sq8_decode.h"

namespace model {

namespace {

template <typename T>
hipError_t alloc_zeroed(T** p, size_t count) {
  hipError_t e = hipMalloc(reinterpret_cast<void**>(p), std::max<size_t>(count, 1) * sizeof(T));
  if (e == hipSuccess) e = hipMemset(*p, 0, std::max<size_t>(count, 1) * sizeof(T));
  return e;
}

template <typename T>
hipError_t alloc_pinned(T** p, size_t count) {
  return hipHostMalloc(reinterpret_cast<void**>(p), std::max<size_t>(count, 1) * sizeof(T),
                       hipHostMallocDefault);
}

}  // namespace

PagedBatchModel::PagedBatchModel(const BatchModelConfig& cfg, const BatchModelWeights& weights,
                                 int max_rows, int max_seq_len, int num_blocks, int block_size,
                                 hipStream_t stream, bool use_graphs, bool split_kv)
    : cfg_(cfg),
      w_(weights),
      max_rows_(max_rows),
      max_seq_len_(max_seq_len),
      num_blocks_(num_blocks),
      block_size_(block_size),
      max_blocks_per_seq_(block_size > 0 ? (max_seq_len + block_size - 1) / block_size : 0),
      use_graphs_(use_graphs),
      split_kv_(split_kv),
      stream_(stream) {}

PagedBatchModel::~PagedBatchModel() {
  if (stream_) (void)hipStreamSynchronize(stream_);
  for (auto& g : graphs_) (void)hipGraphExecDestroy(g.second);
  if (staged_) (void)hipEventDestroy(staged_);
  for (void* p : {static_cast<void*>(kcache_), static_cast<void*>(vcache_),
                  static_cast<void*>(sin_), static_cast<void*>(cos_), static_cast<void*>(x_),
                  static_cast<void*>(qkv_), static_cast<void*>(att_), static_cast<void*>(proj_),
                  static_cast<void*>(gu_), static_cast<void*>(hid_), static_cast<void*>(xn_),
                  static_cast<void*>(logits_), static_cast<void*>(tok_d_),
                  static_cast<void*>(pos_d_), static_cast<void*>(table_d_),
                  static_cast<void*>(next_d_), ws_, att_ws_})
    if (p) (void)hipFree(p);
  for (void* p : {static_cast<void*>(tok_h_), static_cast<void*>(pos_h_),
                  static_cast<void*>(table_h_), static_cast<void*>(next_h_)})
    if (p) (void)hipHostFree(p);
  if (owns_stream_ && stream_) (void)hipStreamDestroy(stream_);
}

size_t PagedBatchModel::kv_pool_bytes() const {
  return 2 * sizeof(float) * static_cast<size_t>(cfg_.layer_num) * num_blocks_ * block_size_ *
         kv_dim_;
}

base::Status PagedBatchModel::check(int rc, const char* what) const {
  if (rc == SQ8_OK) return base::error::Success();
  return base::error::InternalError(std::string(what) + ": " + sq8_status_string(rc));
}

base::Status PagedBatchModel::init() {
  const BatchModelConfig& c = cfg_;
  const int L = c.layer_num;
  if (c.dim <= 0 || c.hidden_dim <= 0 || L <= 0 || c.head_num <= 0 || c.kv_head_num <= 0 ||
      c.vocab_size <= 0 || c.group_size <= 0 || c.dim % c.head_num != 0 ||
      c.head_num % c.kv_head_num != 0)
    return base::error::InvalidArgument("model configuration");
  if (max_rows_ <= 0 || max_seq_len_ <= 0 || num_blocks_ <= 0 || block_size_ <= 0)
    return base::error::InvalidArgument("batch sizes");
  const size_t nl = static_cast<size_t>(L);
  if (w_.qkv.size() != nl || w_.o.size() != nl || w_.gu.size() != nl || w_.down.size() != nl ||
      w_.norm.size() != 2 * nl + 1 || !w_.embedding || !w_.cls.q || !w_.cls.s)
    return base::error::InvalidArgument("weights do not match the layer count");
  for (const auto* v : {&w_.qkv, &w_.o, &w_.gu, &w_.down})
    for (const QuantWeight& q : *v)
      if (!q.q || !q.s) return base::error::InvalidArgument("missing projection weight");
  for (const float* n : w_.norm)
    if (!n) return base::error::InvalidArgument("missing norm weight");
  head_size_ = c.dim / c.head_num;
  kv_dim_ = c.kv_head_num * head_size_;
  // The weights may still be in flight on the caller's streams; the model runs on its own.
  if (hipDeviceSynchronize() != hipSuccess) return base::error::InternalError("device");
  if (!stream_) {
    if (hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking) != hipSuccess)
      return base::error::InternalError("stream creation");
    owns_stream_ = true;
  }
  const size_t R = max_rows_, d = c.dim, kv = kv_dim_, h = c.hidden_dim;
  const size_t layer_elems = static_cast<size_t>(num_blocks_) * block_size_ * kv;
  hipError_t e = hipSuccess;
  auto A = [&](hipError_t r) {
    if (e == hipSuccess) e = r;
  };
  A(alloc_zeroed(&kcache_, nl * layer_elems));
  A(alloc_zeroed(&vcache_, nl * layer_elems));
  A(alloc_zeroed(&sin_, static_cast<size_t>(max_seq_len_) * head_size_));
  A(alloc_zeroed(&cos_, static_cast<size_t>(max_seq_len_) * head_size_));
  A(alloc_zeroed(&x_, R * d));
  A(alloc_zeroed(&xn_, R * d));
  A(alloc_zeroed(&qkv_, R * (d + 2 * kv)));
  A(alloc_zeroed(&att_, R * d));
  A(alloc_zeroed(&proj_, R * d));
  A(alloc_zeroed(&gu_, R * 2 * h));
  A(alloc_zeroed(&hid_, R * h));
  A(alloc_zeroed(&logits_, R * static_cast<size_t>(c.vocab_size)));
  A(alloc_zeroed(&tok_d_, R));
  A(alloc_zeroed(&pos_d_, R));
  A(alloc_zeroed(&table_d_, R * max_blocks_per_seq_));
  A(alloc_zeroed(&next_d_, R));
  A(alloc_pinned(&tok_h_, R));
  A(alloc_pinned(&pos_h_, R));
  A(alloc_pinned(&table_h_, R * max_blocks_per_seq_));
  A(alloc_pinned(&next_h_, R));
  A(hipEventCreateWithFlags(&staged_, hipEventDisableTiming));
  if (e != hipSuccess) return base::error::InternalError(std::string("allocation: ") +
                                                          hipGetErrorString(e));
  // One matmul workspace for every row count, projection and epilogue (graphs keep its
  // address), zeroed once: the split-K tickets start at zero and every call leaves them so.
  const int shapes[5][2] = {{c.dim + 2 * kv_dim_, c.dim}, {c.dim, c.dim},
                            {2 * c.hidden_dim, c.dim}, {c.dim, c.hidden_dim},
                            {c.vocab_size, c.dim}};
  size_t need = 0;
  for (int B = 1; B <= max_rows_; ++B)
    for (const auto& s : shapes)
      for (int epi : {SQ8_EPI_NONE, SQ8_EPI_RESIDUAL, SQ8_EPI_SWIGLU}) {
        const int gs = c.group_size;
        need = std::max(need, w_.packed
                                  ? sq8_epilogue_packed_workspace_bytes(B, s[0], s[1], gs, epi)
                                  : sq8_epilogue_workspace_bytes(B, s[0], s[1], gs, epi));
        if (epi != SQ8_EPI_RESIDUAL)
          need = std::max(need, w_.packed
                                    ? sq8_rmsnorm_rows_packed_workspace_bytes(B, s[0], s[1], gs,
                                                                              epi)
                                    : sq8_rmsnorm_rows_workspace_bytes(B, s[0], s[1], gs, epi));
      }
  ws_bytes_ = need;
  if (need > 0) {
    A(hipMalloc(&ws_, need));
    A(hipMemset(ws_, 0, need));
  }
  if (split_kv_) {
    att_ws_bytes_ = sq8_paged_attention_workspace_bytes(max_rows_, c.head_num, c.kv_head_num,
                                                        head_size_, max_blocks_per_seq_,
                                                        block_size_);
    if (att_ws_bytes_ > 0) {
      A(hipMalloc(&att_ws_, att_ws_bytes_));
      A(hipMemset(att_ws_, 0, att_ws_bytes_));
    }
  }
  if (e != hipSuccess) return base::error::InternalError(std::string("workspace: ") +
                                                          hipGetErrorString(e));
  base::Status st = check(sq8_rope_tables(sin_, cos_, head_size_, max_seq_len_, c.rope_theta,
                                          stream_),
                          "rope tables");
  if (!st) return st;
  if (hipStreamSynchronize(stream_) != hipSuccess)
    return base::error::InternalError("initialisation");
  ready_ = true;
  return base::error::Success();
}

int PagedBatchModel::matmul(const float* x, QuantWeight w, float* y, int M, int N, int K) {
  return w_.packed ? sq8_matmul_packed(x, w.q, w.s, y, M, N, K, cfg_.group_size, ws_, ws_bytes_,
                                       stream_)
                   : sq8_matmul(x, w.q, w.s, y, M, N, K, cfg_.group_size, ws_, ws_bytes_,
                                stream_);
}

int PagedBatchModel::matmul_epilogue(const float* x, QuantWeight w, float* y, int M, int N,
                                     int K, int epi, const float* residual) {
  return w_.packed ? sq8_matmul_epilogue_packed(x, w.q, w.s, y, M, N, K, cfg_.group_size, epi,
                                                residual, ws_, ws_bytes_, stream_)
                   : sq8_matmul_epilogue(x, w.q, w.s, y, M, N, K, cfg_.group_size, epi,
                                         residual, ws_, ws_bytes_, stream_);
}

int PagedBatchModel::matmul_norm(float* x, const float* res, const float* norm_w, QuantWeight w,
                                 float* y, int M, int N, int K, int epi) {
  return w_.packed ? sq8_matmul_rmsnorm_rows_packed(x, res, norm_w, cfg_.eps, w.q, w.s, y, M, N,
                                                    K, cfg_.group_size, epi, ws_, ws_bytes_,
                                                    stream_)
                   : sq8_matmul_rmsnorm_rows(x, res, norm_w, cfg_.eps, w.q, w.s, y, M, N, K,
                                             cfg_.group_size, epi, ws_, ws_bytes_, stream_);
}

base::Status PagedBatchModel::launch(int B, int nd) {
  const BatchModelConfig& c = cfg_;
  const int L = c.layer_num, d = c.dim, kv = kv_dim_, h = c.hidden_dim, gs = c.group_size;
  const size_t layer_elems = static_cast<size_t>(num_blocks_) * block_size_ * kv;
  const bool pk = w_.packed;
  const bool fuse_o = pk ? sq8_epilogue_packed_fused(B, d, d, gs) : sq8_epilogue_fused(B, d, d, gs);
  const bool fuse_gu = pk ? sq8_epilogue_packed_fused(B, 2 * h, d, gs)
                          : sq8_epilogue_fused(B, 2 * h, d, gs);
  const bool fuse_down = pk ? sq8_epilogue_packed_fused(B, d, h, gs)
                            : sq8_epilogue_fused(B, d, h, gs);
  int rc = sq8_embedding(w_.embedding, c.vocab_size, d, tok_d_, B, x_, stream_);
  if (rc) return check(rc, "embedding");
  bool pending = false;  // proj_ holds the FFN output still to be added to x_
  for (int l = 0; l < L; ++l) {
    // residual of the previous FFN (if pending), this layer's attention norm, QKV
    rc = matmul_norm(x_, pending ? proj_ : nullptr, w_.norm[l], w_.qkv[l], qkv_, B, d + 2 * kv,
                     d, SQ8_EPI_NONE);
    if (rc) return check(rc, "qkv");
    float* kc = kcache_ + l * layer_elems;
    float* vc = vcache_ + l * layer_elems;
    rc = sq8_paged_rope_kv(qkv_, B, c.head_num, c.kv_head_num, head_size_, pos_d_, table_d_,
                           max_blocks_per_seq_, block_size_, sin_, cos_, kc, vc, stream_);
    if (rc) return check(rc, "rope + kv write");
    rc = att_ws_ ? sq8_paged_attention_ws(qkv_, d + 2 * kv, B, c.head_num, c.kv_head_num,
                                          head_size_, pos_d_, table_d_, max_blocks_per_seq_,
                                          block_size_, kc, vc, att_, att_ws_, att_ws_bytes_,
                                          stream_)
                 : sq8_paged_attention(qkv_, d + 2 * kv, B, c.head_num, c.kv_head_num,
                                       head_size_, pos_d_, table_d_, max_blocks_per_seq_,
                                       block_size_, kc, vc, att_, stream_);
    if (rc) return check(rc, "attention");
    rc = fuse_o ? matmul_epilogue(att_, w_.o[l], x_, B, d, d, SQ8_EPI_RESIDUAL, x_)
                : matmul(att_, w_.o[l], proj_, B, d, d);
    if (rc) return check(rc, "o");
    const float* gres = fuse_o ? nullptr : proj_;  // residual still to be added before the norm
    if (fuse_gu) {
      rc = matmul_norm(x_, gres, w_.norm[L + l], w_.gu[l], hid_, B, 2 * h, d, SQ8_EPI_SWIGLU);
    } else {
      rc = matmul_norm(x_, gres, w_.norm[L + l], w_.gu[l], gu_, B, 2 * h, d, SQ8_EPI_NONE);
      if (!rc) rc = sq8_swiglu_rows(gu_, B, h, hid_, stream_);
    }
    if (rc) return check(rc, "gate/up");
    if (fuse_down) {
      rc = matmul_epilogue(hid_, w_.down[l], x_, B, d, h, SQ8_EPI_RESIDUAL, x_);
      pending = false;
    } else {
      rc = matmul(hid_, w_.down[l], proj_, B, d, h);
      pending = true;
    }
    if (rc) return check(rc, "down");
  }
  if (nd > 0) {
    rc = pending ? sq8_add_rmsnorm(x_, proj_, w_.norm[2 * L], xn_, nd, d, c.eps, stream_)
                 : sq8_rmsnorm(x_, w_.norm[2 * L], xn_, nd, d, c.eps, stream_);
    if (rc) return check(rc, "final norm");
    rc = matmul(xn_, w_.cls, logits_, nd, c.vocab_size, d);
    if (rc) return check(rc, "classifier");
    rc = sq8_argmax_rows(logits_, nd, c.vocab_size, next_d_, stream_);
    if (rc) return check(rc, "argmax");
  }
  return base::error::Success();
}

base::Status PagedBatchModel::capture(int B) {
  hipGraph_t g = nullptr;
  if (hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal) != hipSuccess)
    return base::error::InternalError("begin capture");
  base::Status st = launch(B, B);
  const hipError_t e = hipStreamEndCapture(stream_, &g);
  if (!st) {
    if (g) (void)hipGraphDestroy(g);
    return st;
  }
  if (e != hipSuccess || !g) return base::error::InternalError("end capture");
  hipGraphExec_t exec = nullptr;
  const hipError_t ei = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (ei != hipSuccess) return base::error::InternalError("graph instantiation");
  graphs_[B] = exec;
  return base::error::Success();
}

base::Status PagedBatchModel::capture_decode_graphs() {
  if (!ready_) return base::error::InternalError("init() not called");
  if (rows_run_ > 0)
    return base::error::InvalidArgument(
        "capture_decode_graphs after a forward step would overwrite block 0 of the KV cache");
  for (int B = 1; B <= max_rows_; ++B) {
    if (graphs_.count(B)) continue;
    // Placeholder rows: token 0 at position 0 of physical block 0.
    hipError_t e = hipMemsetAsync(tok_d_, 0, B * sizeof(int32_t), stream_);
    if (e == hipSuccess) e = hipMemsetAsync(pos_d_, 0, B * sizeof(int32_t), stream_);
    if (e == hipSuccess)
      e = hipMemsetAsync(table_d_, 0, static_cast<size_t>(B) * max_blocks_per_seq_ *
                                          sizeof(int32_t), stream_);
    if (e != hipSuccess) return base::error::InternalError("placeholder rows");
    base::Status st = launch(B, B);
    if (!st) return st;
    st = capture(B);
    if (!st) return st;
  }
  return hipStreamSynchronize(stream_) == hipSuccess ? base::error::Success()
                                                      : base::error::InternalError("capture");
}

base::Status PagedBatchModel::forward_batch(int batch, int nd, const int32_t* tokens,
                                            const int32_t* positions, const int32_t* seq_ids,
                                            const int32_t* block_table, int table_stride,
                                            int32_t* next_tokens) {
  (void)seq_ids;
  if (!ready_) return base::error::InternalError("init() not called");
  if (batch <= 0 || batch > max_rows_ || nd < 0 || nd > batch)
    return base::error::InvalidArgument("row count");
  if (table_stride != max_blocks_per_seq_)
    return base::error::InvalidArgument("block-table width does not match the model");
  for (int i = 0; i < batch; ++i) {
    if (positions[i] < 0 || positions[i] >= max_seq_len_ || tokens[i] < 0 ||
        tokens[i] >= cfg_.vocab_size)
      return base::error::InvalidArgument("row token or position out of range");
    // Attention reads blocks 0 .. pos / block_size of the row's table: all must be mapped.
    const int32_t* t = block_table + static_cast<size_t>(i) * table_stride;
    for (int j = 0; j <= positions[i] / block_size_; ++j)
      if (t[j] < 0 || t[j] >= num_blocks_)
        return base::error::InvalidArgument("row position has no cache block");
  }
  // The pinned staging buffers are free once the previous step's uploads are done (a step
  // without decode rows returns without waiting for its kernels).
  if (hipEventSynchronize(staged_) != hipSuccess) return base::error::InternalError("stream");
  std::memcpy(tok_h_, tokens, batch * sizeof(int32_t));
  std::memcpy(pos_h_, positions, batch * sizeof(int32_t));
  std::memcpy(table_h_, block_table, static_cast<size_t>(batch) * table_stride * sizeof(int32_t));
  hipError_t e = hipMemcpyAsync(tok_d_, tok_h_, batch * sizeof(int32_t),
                                hipMemcpyHostToDevice, stream_);
  if (e == hipSuccess)
    e = hipMemcpyAsync(pos_d_, pos_h_, batch * sizeof(int32_t), hipMemcpyHostToDevice, stream_);
  if (e == hipSuccess)
    e = hipMemcpyAsync(table_d_, table_h_,
                       static_cast<size_t>(batch) * table_stride * sizeof(int32_t),
                       hipMemcpyHostToDevice, stream_);
  if (e == hipSuccess) e = hipEventRecord(staged_, stream_);
  if (e != hipSuccess) return base::error::InternalError("input upload");
  const bool decode_only = nd == batch;
  const auto g = use_graphs_ && decode_only ? graphs_.find(batch) : graphs_.end();
  if (g != graphs_.end()) {
    if (hipGraphLaunch(g->second, stream_) != hipSuccess)
      return base::error::InternalError("graph launch");
    ++graph_replays_;
  } else {
    base::Status st = launch(batch, nd);
    if (!st) return st;
    if (use_graphs_ && decode_only) {
      st = capture(batch);
      if (!st) return st;
    }
  }
  rows_run_ += batch;
  if (nd == 0) return base::error::Success();
  e = hipMemcpyAsync(next_h_, next_d_, nd * sizeof(int32_t), hipMemcpyDeviceToHost, stream_);
  if (e == hipSuccess) e = hipStreamSynchronize(stream_);
  if (e != hipSuccess) return base::error::InternalError(std::string("step: ") +
                                                          hipGetErrorString(e));
  std::memcpy(next_tokens, next_h_, nd * sizeof(int32_t));
  return base::error::Success();
}

}  // namespace model
