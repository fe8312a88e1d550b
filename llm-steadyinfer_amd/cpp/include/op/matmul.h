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

  // Opt-in packed weights (no reference counterpart; the reference keeps the row-major upload of
  // LayerParam::to_cuda, src/source/op/layer.cpp:174-182). With set_packed_weights(true) before
  // to_cuda, or pack_weights() on a layer whose weight is already on the device, the weight is
  // rewritten once into the sq8_pack_weights layout and only the packed copy is kept; forward()
  // then runs kernel::get_matmul_kernel_quant8_packed. Results: bit-identical to the row-major
  // kernels from 3 token rows on, the same tolerance to the reference at 1-2 rows (sq8.h).
  // Quantised HIP layers only; K % 64 == 0 and the group size a multiple of 64.
  void set_packed_weights(bool packed) { pack_on_upload_ = packed; }
  base::Status pack_weights();
  bool weights_packed() const { return weights_packed_; }

  void set_batch_size(int32_t batch) { batch_size_ = batch; }
  int32_t batch_size() const { return batch_size_; }

 private:
  int32_t dim0_ = 0;
  int32_t dim1_ = 0;
  int32_t batch_size_ = 1;
  bool has_bias_ = false;
  bool pack_on_upload_ = false;
  bool weights_packed_ = false;
  std::vector<tensor::Tensor> bias_;
};

}  // namespace op
#endif  // SQ8_OP_OP_MATMUL_H_
