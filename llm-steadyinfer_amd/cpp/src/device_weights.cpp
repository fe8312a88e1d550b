// Upload of an INT8 model file's weights for the native models (model/device_weights.h).
#include "model/device_weights.h"

#include <algorithm>

#include "../../../include/sq8.h"

namespace model {

DeviceWeights::~DeviceWeights() {
  for (void* p : bufs_) (void)hipFree(p);
}

void* DeviceWeights::alloc(size_t bytes, hipError_t* e) {
  void* p = nullptr;
  if (*e == hipSuccess) *e = hipMalloc(&p, bytes);
  if (*e == hipSuccess) bufs_.push_back(p);
  return p;
}

// Rows of `parts` stacked in order into one [sum N][K] int8 weight, their scales concatenated.
base::Status DeviceWeights::fused(const std::vector<const op::MatmulLayer*>& parts, bool packed,
                                  hipStream_t stream, QuantWeight* out) {
  const tensor::Tensor& w0 = parts.front()->get_weight(0);
  const int K = w0.get_dim(1);
  int N = 0;
  for (const op::MatmulLayer* m : parts) {
    const tensor::Tensor& w = m->get_weight(0);
    if (w.dims_size() != 2 || w.get_dim(1) != K || w.data_type() != base::DataType::kDataTypeInt8)
      return base::error::InvalidArgument("fused projections must share their input width");
    N += w.get_dim(0);
  }
  const int gs = parts.front()->group_size();
  if (gs <= 0 || K % gs != 0) return base::error::InvalidArgument("group size");
  const size_t qbytes = static_cast<size_t>(N) * K;
  const size_t sbytes = qbytes / gs * sizeof(float);
  hipError_t e = hipSuccess;
  int8_t* q = static_cast<int8_t*>(alloc(qbytes, &e));
  float* s = static_cast<float*>(alloc(sbytes, &e));
  size_t qo = 0, so = 0;
  for (const op::MatmulLayer* m : parts) {
    const tensor::Tensor& w = m->get_weight(0);
    const tensor::Tensor& sc = m->get_scales();
    if (e == hipSuccess)
      e = hipMemcpyAsync(q + qo, w.ptr<int8_t>(), w.byte_size(), hipMemcpyHostToDevice, stream);
    if (e == hipSuccess)
      e = hipMemcpyAsync(reinterpret_cast<char*>(s) + so, sc.ptr<float>(), sc.byte_size(),
                         hipMemcpyHostToDevice, stream);
    qo += w.byte_size();
    so += sc.byte_size();
  }
  if (e != hipSuccess) return base::error::InternalError("weight upload");
  if (qo != qbytes || so != sbytes) return base::error::InternalError("scale count");
  if (packed) {
    int8_t* p = static_cast<int8_t*>(alloc(sq8_packed_weight_bytes(N, K), &e));
    if (e != hipSuccess) return base::error::InternalError("packed weight allocation");
    const int rc = sq8_pack_weights(q, N, K, p, stream);
    if (rc != SQ8_OK) return base::error::InternalError(std::string("repack: ") +
                                                        sq8_status_string(rc));
    // The row-major copy is freed once the repack has read it (below, after the sync).
    out->q = p;
  } else {
    out->q = q;
  }
  out->s = s;
  return base::error::Success();
}

base::Status DeviceWeights::upload(const Int8ModelFile& file, bool packed, hipStream_t stream) {
  QuantLayers ql;
  base::Status st = file.create_quant_layers(base::DeviceType::kDeviceCPU, &ql);
  if (!st) return st;
  const TransformerConfig& tc = file.config();
  cfg_.dim = tc.dim_;
  cfg_.hidden_dim = tc.hidden_dim_;
  cfg_.layer_num = tc.layer_num_;
  cfg_.head_num = tc.head_num_;
  cfg_.kv_head_num = tc.kv_head_num_;
  cfg_.vocab_size = tc.vocab_size_;
  cfg_.rope_theta = tc.rope_theta_;
  cfg_.group_size = file.group_size();
  w_ = BatchModelWeights();
  w_.packed = packed;
  const int L = tc.layer_num_;
  w_.qkv.resize(L);
  w_.o.resize(L);
  w_.gu.resize(L);
  w_.down.resize(L);
  for (int l = 0; l < L; ++l) {
    st = fused({ql.wq[l].get(), ql.wk[l].get(), ql.wv[l].get()}, packed, stream, &w_.qkv[l]);
    if (st) st = fused({ql.wo[l].get()}, packed, stream, &w_.o[l]);
    if (st) st = fused({ql.w1[l].get(), ql.w3[l].get()}, packed, stream, &w_.gu[l]);
    if (st) st = fused({ql.w2[l].get()}, packed, stream, &w_.down[l]);
    if (!st) return st;
  }
  st = fused({ql.cls.get()}, packed, stream, &w_.cls);
  if (!st) return st;
  hipError_t e = hipSuccess;
  const size_t emb = static_cast<size_t>(tc.vocab_size_) * tc.dim_ * sizeof(float);
  float* embd = static_cast<float*>(alloc(emb, &e));
  if (e == hipSuccess)
    e = hipMemcpyAsync(embd, ql.embedding, emb, hipMemcpyHostToDevice, stream);
  w_.embedding = embd;
  for (const float* n : ql.rmsnorm) {
    float* nd = static_cast<float*>(alloc(tc.dim_ * sizeof(float), &e));
    if (e == hipSuccess)
      e = hipMemcpyAsync(nd, n, tc.dim_ * sizeof(float), hipMemcpyHostToDevice, stream);
    w_.norm.push_back(nd);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return base::error::InternalError(std::string("upload: ") +
                                                          hipGetErrorString(e));
  if (packed) {  // drop the row-major copies the repacks read
    std::vector<void*> keep;
    std::vector<const void*> live;
    for (const auto* v : {&w_.qkv, &w_.o, &w_.gu, &w_.down})
      for (const QuantWeight& q : *v) live.push_back(q.q), live.push_back(q.s);
    live.push_back(w_.cls.q);
    live.push_back(w_.cls.s);
    live.push_back(w_.embedding);
    for (const float* n : w_.norm) live.push_back(n);
    for (void* p : bufs_) {
      if (std::find(live.begin(), live.end(), p) != live.end())
        keep.push_back(p);
      else
        (void)hipFree(p);
    }
    bufs_.swap(keep);
  }
  return base::error::Success();
}

}  // namespace model
