// Kernel dispatch of the op API for the quantised matmul. Mirrors the reference's
// src/source/op/kernels/kernels_interface.h:12-14 (MatmulKernelQuant) and
// src/source/op/kernels/kernels_interfaces.cpp:54-61 (get_matmul_kernel_quant8): the HIP device
// returns matmul_kernel_hip_qint8, which runs the gfx950 kernels through the C ABI (sq8.h); any
// other device is a fatal error, as in the reference (there is no CPU INT8 matmul).
#ifndef SQ8_OP_KERNELS_KERNELS_INTERFACE_H_
#define SQ8_OP_KERNELS_KERNELS_INTERFACE_H_
#include "base/hip_config.h"
#include "tensor/tensor.h"

namespace kernel {

typedef void (*MatmulKernelQuant)(const tensor::Tensor& input, const tensor::Tensor& weight,
                                  const tensor::Tensor& output, int32_t group_size,
                                  const tensor::Tensor& scale, const HipConfig* config);

typedef void (*AddKernel)(const tensor::Tensor& input1, const tensor::Tensor& input2,
                          const tensor::Tensor& output, void* stream);

// input [batch*K] fp32, weight int8 [N, K], scale fp32 [N*K/group_size], output [batch*N] fp32,
// all on the device. Launches asynchronously on config->stream; aborts on invalid arguments or a
// failed launch (the reference CHECKs the same conditions, matmul_kernel.cu:165-185).
void matmul_kernel_hip_qint8(const tensor::Tensor& input, const tensor::Tensor& weight,
                             const tensor::Tensor& output, int32_t group_size,
                             const tensor::Tensor& scale, const HipConfig* config);

// output[b, :] = input1[b, :] + input2 for a [K] bias broadcast over rows (device tensors).
void add_kernel_hip(const tensor::Tensor& input1, const tensor::Tensor& input2,
                    const tensor::Tensor& output, void* stream);

MatmulKernelQuant get_matmul_kernel_quant8(base::DeviceType device_type);

// As matmul_kernel_hip_qint8 with the weight in the sq8_pack_weights layout (the tensor keeps
// dims [N, K]; its buffer holds whole 16-row tiles): sq8_matmul_packed. No reference
// counterpart: MatmulLayer's opt-in packed upload dispatches here.
void matmul_kernel_hip_qint8_packed(const tensor::Tensor& input, const tensor::Tensor& weight,
                                    const tensor::Tensor& output, int32_t group_size,
                                    const tensor::Tensor& scale, const HipConfig* config);
MatmulKernelQuant get_matmul_kernel_quant8_packed(base::DeviceType device_type);
AddKernel get_add_kernel(base::DeviceType device_type);

}  // namespace kernel
#endif  // SQ8_OP_KERNELS_KERNELS_INTERFACE_H_
