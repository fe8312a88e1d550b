// Device copies of an INT8 model file's weights in the layout the native models
// (model::PagedBatchModel, model::Int8Decoder) take: the reference uploads each MatmulLayer on
// its own (LayerParam::to_cuda, src/source/op/layer.cpp:174-182); here the projections that read
// the same input are fused at upload, QKV = [wq; wk; wv] and gate/up = [w1; w3] (rows stacked,
// scales concatenated in the same order; each output row is unchanged because groups never cross
// rows), and with `packed` each projection is repacked once (sq8_pack_weights) and only the
// packed copy is kept. The embedding and the 2L + 1 RMSNorm weights are copied as they are.
#ifndef SQ8_OP_MODEL_DEVICE_WEIGHTS_H_
#define SQ8_OP_MODEL_DEVICE_WEIGHTS_H_
#include <hip/hip_runtime.h>

#include <vector>

#include "base/base.h"
#include "model/int8_model_file.h"
#include "model/paged_batch_model.h"

namespace model {

class DeviceWeights {
 public:
  DeviceWeights() = default;
  DeviceWeights(const DeviceWeights&) = delete;
  DeviceWeights& operator=(const DeviceWeights&) = delete;
  ~DeviceWeights();

  // Reads the file's projections (Int8ModelFile::create_quant_layers on the host) and uploads
  // them; returns when the copies are complete.
  base::Status upload(const Int8ModelFile& file, bool packed, hipStream_t stream = nullptr);

  const BatchModelWeights& weights() const { return w_; }
  // The model's shape from the file header, with the file's group size.
  const BatchModelConfig& config() const { return cfg_; }

 private:
  base::Status fused(const std::vector<const op::MatmulLayer*>& parts, bool packed,
                     hipStream_t stream, QuantWeight* out);
  void* alloc(size_t bytes, hipError_t* e);

  std::vector<void*> bufs_;
  BatchModelWeights w_;
  BatchModelConfig cfg_;
};

}  // namespace model
#endif  // SQ8_OP_MODEL_DEVICE_WEIGHTS_H_
