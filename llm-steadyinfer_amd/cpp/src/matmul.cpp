// MatmulLayer (reference: src/source/op/matmul.cpp:19-195).
#include "op/matmul.h"
#include "kernels/kernels_interface.h"
#include "../../../include/sq8.h"

namespace op {

MatmulLayer::MatmulLayer(base::DeviceType device_type, int32_t dim0, int32_t dim1,
                         bool is_quant_layer, bool has_bias)
    : LayerParam(device_type, LayerType::kLayerMatmul, is_quant_layer, "Matmul"),
      dim0_(dim0),
      dim1_(dim1),
      has_bias_(has_bias) {
  reset_input_size(1);
  reset_output_size(1);
  reset_weight_size(1);
  if (has_bias_) bias_.resize(1);
}

base::Status MatmulLayer::check() const {
  const auto& input = get_input(0);
  const bool batched = input.dims_size() == 2;
  base::Status st =
      batched ? check_tensor_with_dim(input, device_type_, data_type_, {input.get_dim(0), dim1_})
              : check_tensor_with_dim(input, device_type_, data_type_, {dim1_});
  if (!st) {
    LOG_ERROR << "The input tensor error in the matmul layer.";
    return st;
  }
  st = check_tensor_with_dim(get_weight(0), device_type_,
                             is_quant_layer_ ? base::DataType::kDataTypeInt8 : data_type_,
                             {dim0_, dim1_});
  if (!st) {
    LOG_ERROR << "The weight tensor error in the matmul layer.";
    return st;
  }
  if (is_quant_layer_) {
    st = check_tensor_with_dim(scales_, device_type_, base::DataType::kDataTypeFp32,
                               {static_cast<int32_t>(scales_.size())});
    if (!st) {
      LOG_ERROR << "The scale tensor error in the matmul layer.";
      return st;
    }
  }
  const auto& output = get_output(0);
  st = batched ? check_tensor_with_dim(output, device_type_, data_type_, {input.get_dim(0), dim0_})
               : check_tensor_with_dim(output, device_type_, data_type_, {dim0_});
  if (!st) {
    LOG_ERROR << "The output tensor error in the matmul layer.";
    return st;
  }
  return base::error::Success();
}

base::Status MatmulLayer::forward() {
  base::Status st = check();
  if (!st) return st;
  if (device_type_ == base::DeviceType::kDeviceHIP) CHECK(cuda_config_ != nullptr);
  const auto& input = get_input(0);
  const int32_t batch = input.dims_size() == 2 ? input.get_dim(0) : 1;
  auto& output = get_output(0);
  // Flat views [batch*dim1] and [batch*dim0], as the reference hands them to the kernel.
  tensor::Tensor input_flat(base::DataType::kDataTypeFp32, batch * dim1_, false, nullptr,
                            const_cast<float*>(input.ptr<float>()));
  input_flat.set_device_type(device_type_);
  tensor::Tensor output_flat(base::DataType::kDataTypeFp32, batch * dim0_, false, nullptr,
                             output.ptr<float>());
  output_flat.set_device_type(device_type_);
  if (!is_quant_layer_)
    return base::error::FunctionNotImplement("fp32 weights are served by the reference's GEMM");
  const kernel::MatmulKernelQuant kern =
      weights_packed_ ? kernel::get_matmul_kernel_quant8_packed(device_type_)
                      : kernel::get_matmul_kernel_quant8(device_type_);
  kern(input_flat, get_weight(0), output_flat, group_size_, scales_, cuda_config_.get());
  if (has_bias_) {
    kernel::get_add_kernel(device_type_)(output_flat, get_bias(0), output_flat,
                                         cuda_config_ ? cuda_config_->stream : nullptr);
  }
  return base::error::Success();
}

// The bias is fp32 [dim] for quantised and fp32 layers alike. (The reference's quantised branch,
// matmul.cpp:155-170, would bind an int8 bias and replace the layer's weight scales with the
// bias's trailing block; no reference loader calls it on a quantised layer.)
base::Status MatmulLayer::set_bias(int32_t idx, int32_t& dim, const void* bias_ptr,
                                   base::DeviceType device_type) {
  CHECK_GE(idx, 0);
  CHECK_LT(static_cast<size_t>(idx), bias_.size());
  CHECK(bias_ptr != nullptr);
  auto buffer = std::make_shared<base::Buffer>(static_cast<size_t>(dim) * sizeof(float), nullptr,
                                               const_cast<void*>(bias_ptr), true);
  if (device_type != base::DeviceType::kDeviceUnknown) buffer->set_device_type(device_type);
  tensor::Tensor bias(base::DataType::kDataTypeFp32, dim);
  CHECK(bias.assign(buffer));
  bias_[idx] = bias;
  return base::error::Success();
}

tensor::Tensor& MatmulLayer::get_bias(int32_t idx) {
  CHECK_GE(idx, 0);
  CHECK_LT(static_cast<size_t>(idx), bias_.size());
  return bias_[idx];
}

const tensor::Tensor& MatmulLayer::get_bias(int32_t idx) const {
  CHECK_GE(idx, 0);
  CHECK_LT(static_cast<size_t>(idx), bias_.size());
  return bias_[idx];
}

void MatmulLayer::to_cuda() {
  LayerParam::to_cuda();
  hipStream_t st = cuda_config_ ? cuda_config_->stream : nullptr;
  for (auto& b : bias_)
    if (!b.is_empty()) b.to_cuda(st);
  if (pack_on_upload_ && !weights_packed_) {
    const base::Status s = pack_weights();
    CHECK(s) << "packed weight upload: " << s.get_err_msg();
  }
}

base::Status MatmulLayer::pack_weights() {
  if (weights_packed_) return base::error::Success();
  if (!is_quant_layer_) return base::error::InvalidArgument("packed weights need a quantised layer");
  const tensor::Tensor& w = get_weight(0);
  if (w.is_empty() || w.dims_size() != 2 || w.device_type() != base::DeviceType::kDeviceHIP)
    return base::error::InvalidArgument("packed weights need the [dim0, dim1] weight on the device");
  const int32_t N = w.get_dim(0), K = w.get_dim(1);
  if (N != dim0_ || K != dim1_ || K % 64 != 0 || group_size_ <= 0 || group_size_ % 64 != 0 ||
      K % group_size_ != 0)
    return base::error::InvalidArgument("packed weights need K % 64 == 0 and a group size that is "
                                        "a multiple of 64 dividing K");
  auto alloc = base::HIPDeviceAllocatorFactory::get_instance();
  auto buf = std::make_shared<base::Buffer>(sq8_packed_weight_bytes(N, K), alloc);
  if (!buf->ptr()) return base::error::InternalError("packed weight allocation");
  buf->set_device_type(base::DeviceType::kDeviceHIP);
  hipStream_t st = cuda_config_ ? cuda_config_->stream : nullptr;
  const int rc = sq8_pack_weights(w.ptr<int8_t>(), N, K, static_cast<int8_t*>(buf->ptr()), st);
  if (rc != SQ8_OK) return base::error::InternalError(std::string("sq8_pack_weights: ") +
                                                      sq8_status_string(rc));
  // The row-major copy may be released (below) only once the repack has read it.
  if (hipStreamSynchronize(st) != hipSuccess) return base::error::InternalError("repack");
  tensor::Tensor packed(base::DataType::kDataTypeInt8, N, K);
  if (!packed.assign(buf)) return base::error::InternalError("packed weight tensor");
  weights_[0] = packed;  // dims stay [dim0, dim1]; the buffer holds whole 16-row tiles
  weights_packed_ = true;
  return base::error::Success();
}

}  // namespace op
