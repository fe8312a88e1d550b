// Layer base classes (reference: src/source/op/layer.cpp).
#include "op/layer.h"

namespace op {

BaseLayer::BaseLayer(base::DeviceType device_type, LayerType layer_type, base::DataType data_type,
                     std::string layer_name)
    : layer_name_(std::move(layer_name)),
      layer_type_(layer_type),
      data_type_(data_type),
      device_type_(device_type) {}

base::Status BaseLayer::set_weight(int32_t, const tensor::Tensor&) {
  return base::error::FunctionNotImplement();
}

base::Status BaseLayer::set_weight(int32_t, const std::vector<int32_t>&, const void*,
                                   base::DeviceType) {
  return base::error::FunctionNotImplement();
}

Layer::Layer(base::DeviceType device_type, LayerType layer_type, std::string layer_name)
    : BaseLayer(device_type, layer_type, base::DataType::kDataTypeFp32, std::move(layer_name)) {}

base::Status Layer::check_tensor(const tensor::Tensor& t, base::DeviceType device_type,
                                 base::DataType data_type) const {
  if (t.is_empty()) return base::error::InvalidArgument("The tensor parameter is empty.");
  if (t.device_type() != device_type)
    return base::error::InvalidArgument("The tensor has a wrong device type.");
  if (t.data_type() != data_type)
    return base::error::InvalidArgument("The tensor has a wrong data type.");
  return base::error::Success();
}

base::Status Layer::check_tensor_with_dim(const tensor::Tensor& t, base::DeviceType device_type,
                                          base::DataType data_type,
                                          const std::vector<int32_t>& dims) const {
  base::Status st = check_tensor(t, device_type, data_type);
  if (!st) return st;
  if (static_cast<size_t>(t.dims_size()) != dims.size())
    return base::error::InvalidArgument("The tensor has a wrong rank.");
  for (int32_t i = 0; i < t.dims_size(); ++i)
    if (t.get_dim(i) != dims[i])
      return base::error::InvalidArgument("The tensor has a wrong dim in dim" + std::to_string(i));
  return base::error::Success();
}

base::Status Layer::check() const {
  return base::error::FunctionNotImplement("The check function is not implement yet");
}

base::Status Layer::forward() { return base::error::FunctionNotImplement(""); }

base::Status Layer::forward(const tensor::Tensor& input1, const tensor::Tensor& output1) {
  set_input(0, input1);
  set_output(0, output1);
  return forward();
}

base::Status Layer::forward(const tensor::Tensor& input1, const tensor::Tensor& input2,
                            const tensor::Tensor& output1) {
  set_input(0, input1);
  set_input(1, input2);
  set_output(0, output1);
  return forward();
}

void Layer::set_input(int32_t idx, const tensor::Tensor& input) {
  CHECK_GE(idx, 0);
  CHECK_LT(static_cast<size_t>(idx), inputs_.size());
  inputs_[idx] = input;
}

void Layer::set_output(int32_t idx, const tensor::Tensor& output) {
  CHECK_GE(idx, 0);
  CHECK_LT(static_cast<size_t>(idx), outputs_.size());
  outputs_[idx] = output;
}

const tensor::Tensor& Layer::get_input(int32_t idx) const {
  CHECK_GE(idx, 0);
  CHECK_LT(static_cast<size_t>(idx), inputs_.size());
  return inputs_[idx];
}

tensor::Tensor& Layer::get_input(int32_t idx) {
  CHECK_GE(idx, 0);
  CHECK_LT(static_cast<size_t>(idx), inputs_.size());
  return inputs_[idx];
}

const tensor::Tensor& Layer::get_output(int32_t idx) const {
  CHECK_GE(idx, 0);
  CHECK_LT(static_cast<size_t>(idx), outputs_.size());
  return outputs_[idx];
}

tensor::Tensor& Layer::get_output(int32_t idx) {
  CHECK_GE(idx, 0);
  CHECK_LT(static_cast<size_t>(idx), outputs_.size());
  return outputs_[idx];
}

void Layer::to_cuda() {
  hipStream_t st = cuda_config_ ? cuda_config_->stream : nullptr;
  for (auto& t : inputs_)
    if (!t.is_empty()) t.to_cuda(st);
  for (auto& t : outputs_)
    if (!t.is_empty()) t.to_cuda(st);
}

void Layer::set_cuda_config(std::shared_ptr<kernel::HipConfig> config) {
  if (config) cuda_config_ = std::move(config);
}

LayerParam::LayerParam(base::DeviceType device_type, LayerType layer_type, bool is_quant_layer,
                       std::string layer_name)
    : Layer(device_type, layer_type, std::move(layer_name)), is_quant_layer_(is_quant_layer) {}

tensor::Tensor& LayerParam::get_weight(int32_t idx) {
  CHECK_GE(idx, 0);
  CHECK_LT(static_cast<size_t>(idx), weights_.size());
  return weights_[idx];
}

const tensor::Tensor& LayerParam::get_weight(int32_t idx) const {
  CHECK_GE(idx, 0);
  CHECK_LT(static_cast<size_t>(idx), weights_.size());
  return weights_[idx];
}

void LayerParam::to_cuda() {
  Layer::to_cuda();
  hipStream_t st = cuda_config_ ? cuda_config_->stream : nullptr;
  for (auto& w : weights_)
    if (!w.is_empty()) w.to_cuda(st);
  if (!scales_.is_empty()) scales_.to_cuda(st);
}

base::Status LayerParam::set_weight(int32_t idx, const tensor::Tensor& weight) {
  CHECK_GE(idx, 0);
  CHECK_LT(static_cast<size_t>(idx), weights_.size());
  if (!weight.is_empty()) CHECK(weight.device_type() == device_type_);
  weights_[idx] = weight;
  return base::error::Success();
}

base::Status LayerParam::set_weight(int32_t idx, const std::vector<int32_t>& dims,
                                    const void* weight_ptr, base::DeviceType device_type) {
  CHECK_GE(idx, 0);
  CHECK_LT(static_cast<size_t>(idx), weights_.size());
  CHECK(weight_ptr != nullptr);
  size_t numel = 1;
  for (int32_t d : dims) numel *= static_cast<size_t>(d);
  const base::DataType dt =
      is_quant_layer_ ? base::DataType::kDataTypeInt8 : base::DataType::kDataTypeFp32;
  auto buffer = std::make_shared<base::Buffer>(numel * base::DataTypeSize(dt), nullptr,
                                               const_cast<void*>(weight_ptr), true);
  if (device_type != base::DeviceType::kDeviceUnknown) buffer->set_device_type(device_type);
  tensor::Tensor weight(dt, dims);
  CHECK(weight.assign(buffer));
  weights_[idx] = weight;
  if (is_quant_layer_) {
    if (group_size_ <= 0 || numel % static_cast<size_t>(group_size_) != 0)
      return base::error::InvalidArgument("weight size is not a multiple of the group size");
    const int32_t nscales = static_cast<int32_t>(numel / group_size_);
    // The fp32 scales follow the int8 block directly.
    scales_ = tensor::Tensor(base::DataType::kDataTypeFp32, nscales, false, nullptr,
                             reinterpret_cast<float*>(
                                 const_cast<int8_t*>(static_cast<const int8_t*>(weight_ptr)) + numel));
    scales_.set_device_type(device_type);
  }
  return base::error::Success();
}

void LayerParam::set_scales(const tensor::Tensor& scales) {
  CHECK(!scales.is_empty());
  scales_ = scales;
}

int32_t LayerParam::get_scale_num() const {
  CHECK(!scales_.is_empty());
  return static_cast<int32_t>(scales_.size());
}

}  // namespace op
