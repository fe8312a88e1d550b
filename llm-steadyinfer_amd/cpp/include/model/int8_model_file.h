// INT8 model file loader: the part of the reference's Model that maps a quantised .bin file and
// binds its projections to MatmulLayers.
//   open()                 Model::read_model_file + generate_model_infos
//                          (src/source/model/model.cpp:295-383): header, int32 group size, mmap,
//                          weight_data = start of the weights;
//   create_quant_layers()  LLamaModel::create_param_quant_layers (src/source/model/llama3.cpp:
//                          193-297; Qwen2Model's, qwen2.cpp:193-297, walks the same layout): the
//                          byte cursor over wq, wk, wv, wo, w1, w2, w3 (per layer), the classifier
//                          (not advanced past when the header's vocab_size is positive), then the
//                          fp32 embedding and the 2L + 1 RMSNorm weights.
// Each quantised block is int8 [rows][cols] followed by rows*cols/group_size fp32 scales and is
// bound with set_group_size + set_weight exactly as the reference does; the layers stay on the
// host until to_cuda().
#ifndef SQ8_OP_MODEL_INT8_MODEL_FILE_H_
#define SQ8_OP_MODEL_INT8_MODEL_FILE_H_
#include <memory>
#include <string>
#include <vector>
#include "base/base.h"
#include "model/config.h"
#include "op/matmul.h"

namespace model {

// Owns the mapping of a model file (reference: src/include/model/raw_model_data.h:6-24).
struct RawModelDataInt8 {
  RawModelDataInt8() = default;
  RawModelDataInt8(const RawModelDataInt8&) = delete;
  RawModelDataInt8& operator=(const RawModelDataInt8&) = delete;
  ~RawModelDataInt8();
  int32_t fd = -1;
  size_t file_size = 0;
  void* data = nullptr;
  void* weight_data = nullptr;
  // Byte offset from the start of the weights.
  const void* weight(size_t offset) const { return static_cast<const int8_t*>(weight_data) + offset; }
};

// The quantised projections and fp32 tensors of one model file.
struct QuantLayers {
  std::vector<std::shared_ptr<op::MatmulLayer>> wq, wk, wv, wo, w1, w2, w3;
  std::shared_ptr<op::MatmulLayer> cls;
  const float* embedding = nullptr;      // [vocab, dim], host (mapped file)
  std::vector<const float*> rmsnorm;     // 2L + 1 of [dim]: attention, ffn, final
};

class Int8ModelFile {
 public:
  base::Status open(const std::string& path);
  base::Status create_quant_layers(base::DeviceType device_type, QuantLayers* layers) const;

  const TransformerConfig& config() const { return config_; }
  int32_t group_size() const { return group_size_; }
  const RawModelDataInt8* raw() const { return raw_.get(); }
  // Byte offset (from the start of the weights) where the cursor ends after the RMSNorm weights.
  size_t weights_end() const { return weights_end_; }

 private:
  TransformerConfig config_;
  int32_t group_size_ = 0;
  size_t weights_end_ = 0;
  std::shared_ptr<RawModelDataInt8> raw_;
};

}  // namespace model
#endif  // SQ8_OP_MODEL_INT8_MODEL_FILE_H_
