// Layer base classes of the op API. Mirrors the reference's src/include/op/layer.h:25-188:
// BaseLayer (type/device/data type, forward overloads), Layer (inputs/outputs, tensor checks,
// device config) and LayerParam (weights, group-quantised scales).
#ifndef SQ8_OP_OP_LAYER_H_
#define SQ8_OP_OP_LAYER_H_
#include <memory>
#include <string>
#include <vector>
#include "base/base.h"
#include "base/hip_config.h"
#include "tensor/tensor.h"

namespace op {

enum class LayerType : uint8_t {
  kLayerUnknown = 0,
  kLayerLinear = 1,
  kLayerEncode = 2,
  kLayerEmbedding = 3,
  kLayerRMSNorm = 4,
  kLayerMatmul = 5,
  kLayerRoPe = 6,
  kLayerMHA = 7,
  kLayerSoftmax = 8,
  kLayerAdd = 9,
  kLayerSwiGLU = 10,
};

class BaseLayer {
 public:
  explicit BaseLayer(base::DeviceType device_type, LayerType layer_type, base::DataType data_type,
                     std::string layer_name = "");
  virtual ~BaseLayer() = default;

  base::DataType data_type() const { return data_type_; }
  LayerType layer_type() const { return layer_type_; }

  virtual base::Status init() = 0;
  virtual base::Status forward() = 0;
  virtual base::Status forward(const tensor::Tensor& input1, const tensor::Tensor& output1) = 0;
  virtual base::Status forward(const tensor::Tensor& input1, const tensor::Tensor& input2,
                               const tensor::Tensor& output1) = 0;

  virtual void set_input(int32_t idx, const tensor::Tensor& input) = 0;
  virtual void set_output(int32_t idx, const tensor::Tensor& output) = 0;
  virtual size_t input_size() const = 0;
  virtual size_t output_size() const = 0;
  virtual base::Status check() const = 0;
  virtual tensor::Tensor& get_input(int32_t idx) = 0;
  virtual tensor::Tensor& get_output(int32_t idx) = 0;
  virtual const tensor::Tensor& get_input(int32_t idx) const = 0;
  virtual const tensor::Tensor& get_output(int32_t idx) const = 0;

  virtual base::Status set_weight(int32_t idx, const tensor::Tensor& weight);
  virtual base::Status set_weight(int32_t idx, const std::vector<int32_t>& dims,
                                  const void* weight_ptr,
                                  base::DeviceType device_type = base::DeviceType::kDeviceUnknown);

  const std::string& get_layer_name() const { return layer_name_; }
  void set_layer_name(const std::string& name) { layer_name_ = name; }
  base::DeviceType device_type() const { return device_type_; }
  void set_device_type(base::DeviceType t) { device_type_ = t; }

 protected:
  std::string layer_name_;
  LayerType layer_type_ = LayerType::kLayerUnknown;
  base::DataType data_type_ = base::DataType::kDataTypeUnknown;
  base::DeviceType device_type_ = base::DeviceType::kDeviceUnknown;
};

class Layer : public BaseLayer {
 public:
  explicit Layer(base::DeviceType device_type, LayerType layer_type, std::string layer_name = "");

  base::Status init() override { return base::error::Success(); }
  base::Status check_tensor(const tensor::Tensor& tensor, base::DeviceType device_type,
                            base::DataType data_type) const;
  // Checks emptiness, device, data type and each dimension against `dims` (its length must be
  // the tensor's rank).
  base::Status check_tensor_with_dim(const tensor::Tensor& tensor, base::DeviceType device_type,
                                     base::DataType data_type,
                                     const std::vector<int32_t>& dims) const;
  base::Status check() const override;
  base::Status forward() override;
  base::Status forward(const tensor::Tensor& input1, const tensor::Tensor& output1) override;
  base::Status forward(const tensor::Tensor& input1, const tensor::Tensor& input2,
                       const tensor::Tensor& output1) override;

  void set_input(int32_t idx, const tensor::Tensor& input) override;
  void set_output(int32_t idx, const tensor::Tensor& output) override;
  const tensor::Tensor& get_input(int32_t idx) const override;
  const tensor::Tensor& get_output(int32_t idx) const override;
  tensor::Tensor& get_input(int32_t idx) override;
  tensor::Tensor& get_output(int32_t idx) override;
  size_t input_size() const override { return inputs_.size(); }
  size_t output_size() const override { return outputs_.size(); }
  void reset_input_size(size_t size) { inputs_.resize(size); }
  void reset_output_size(size_t size) { outputs_.resize(size); }

  // Moves inputs and outputs to the device (the reference's Layer::to_cuda).
  virtual void to_cuda();
  void set_cuda_config(std::shared_ptr<kernel::HipConfig> config);
  std::shared_ptr<kernel::HipConfig> cuda_config() const { return cuda_config_; }

 protected:
  std::vector<tensor::Tensor> inputs_;
  std::vector<tensor::Tensor> outputs_;
  std::shared_ptr<kernel::HipConfig> cuda_config_;
};

class LayerParam : public Layer {
 public:
  explicit LayerParam(base::DeviceType device_type, LayerType layer_type,
                      bool is_quant_layer = false, std::string layer_name = "");

  size_t weight_size() const { return weights_.size(); }
  void reset_weight_size(size_t size) { weights_.resize(size); }
  tensor::Tensor& get_weight(int32_t idx);
  const tensor::Tensor& get_weight(int32_t idx) const;

  void to_cuda() override;

  base::Status set_weight(int32_t idx, const tensor::Tensor& weight) override;
  // Binds a non-owning view of `dims` elements at weight_ptr. For a quantised layer the weight is
  // int8 and its fp32 scales follow immediately after the int8 block: numel/group_size of them
  // (reference: src/source/op/layer.cpp:184-218). set_group_size must be called first.
  base::Status set_weight(int32_t idx, const std::vector<int32_t>& dims, const void* weight_ptr,
                          base::DeviceType device_type = base::DeviceType::kDeviceUnknown) override;

  void set_scales(const tensor::Tensor& scales);
  void set_group_size(int32_t group_size) { group_size_ = group_size; }
  int32_t group_size() const { return group_size_; }
  int32_t get_scale_num() const;
  const tensor::Tensor& get_scales() const { return scales_; }
  bool is_quant_layer() const { return is_quant_layer_; }

 protected:
  int32_t group_size_ = 0;
  bool is_quant_layer_ = false;
  tensor::Tensor scales_;
  std::vector<tensor::Tensor> weights_;
};

}  // namespace op
#endif  // SQ8_OP_OP_LAYER_H_
