// Matmul layer. Mirrors the reference's src/include/op/matmul.h:6-33 and
// src/source/op/matmul.cpp:19-136: weight [dim0 = outputs, dim1 = inputs], input [dim1] or
// [batch, dim1], output [dim0] or [batch, dim0]; quantised layers dispatch to
// kernel::get_matmul_kernel_quant8(device).
#ifndef SQ8_OP_OP_MATMUL_H_
#define SQ8_OP_OP_MATMUL_H_
#include "op/layer.h"

namespace op {

class MatmulLayer : public LayerParam {
 public:
  explicit MatmulLayer(base::DeviceType device_type, int32_t dim0, int32_t dim1,
                       bool is_quant_layer = false, bool has_bias = false);

  base::Status check() const override;
  base::Status forward() override;
  using Layer::forward;

  // Binds a per-output bias (fp32 [dim]); applied after the product.
  base::Status set_bias(int32_t idx, int32_t& dim, const void* bias_ptr,
                        base::DeviceType device_type);
  tensor::Tensor& get_bias(int32_t idx);
  const tensor::Tensor& get_bias(int32_t idx) const;

  void to_cuda() override;

  void set_batch_size(int32_t batch) { batch_size_ = batch; }
  int32_t batch_size() const { return batch_size_; }

 private:
  int32_t dim0_ = 0;
  int32_t dim1_ = 0;
  int32_t batch_size_ = 1;
  bool has_bias_ = false;
  std::vector<tensor::Tensor> bias_;
};

}  // namespace op
#endif  // SQ8_OP_OP_MATMUL_H_
