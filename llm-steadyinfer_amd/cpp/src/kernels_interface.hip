// Device dispatch for the quantised matmul (reference: src/source/op/kernels/kernels_interfaces.cpp
// :54-61 and matmul_kernel_cu_qint8, src/source/op/kernels/cuda/matmul_kernel.cu:162-196).
#include "kernels/kernels_interface.h"
#include "sq8.h"

namespace kernel {

namespace {
// Shape checks of the reference's launcher (matmul_kernel.cu:165-185) and one sq8 call on
// config->stream with the config's workspace.
template <bool kPacked>
void matmul_qint8(const tensor::Tensor& input, const tensor::Tensor& weight,
                  const tensor::Tensor& output, int32_t group_size, const tensor::Tensor& scale,
                  const HipConfig* config) {
  CHECK(config != nullptr);
  CHECK(!input.is_empty() && input.dims_size() <= 2);
  CHECK(input.device_type() == base::DeviceType::kDeviceHIP);
  CHECK(!weight.is_empty() && weight.dims_size() == 2);
  CHECK(weight.device_type() == base::DeviceType::kDeviceHIP);
  const int32_t N = weight.get_dim(0);  // output rows
  const int32_t K = weight.get_dim(1);  // input width
  const int32_t in_size = static_cast<int32_t>(input.size());
  const int32_t out_size = static_cast<int32_t>(output.size());
  CHECK_EQ(in_size % K, 0);
  CHECK_EQ(out_size % N, 0);
  const int32_t M = in_size / K;
  CHECK_EQ(M, out_size / N);
  auto* cfg = const_cast<HipConfig*>(config);
  const size_t ws_bytes = kPacked ? sq8_packed_workspace_bytes(M, N, K, group_size)
                                  : sq8_workspace_bytes(M, N, K, group_size);
  void* ws = cfg->workspace(ws_bytes);
  CHECK(ws_bytes == 0 || ws != nullptr)
      << "sq8_matmul needs a " << ws_bytes << "-byte workspace, which cannot grow while the stream "
      << "captures a graph (HipConfig::reserve_workspace before the capture)";
  float* y = const_cast<float*>(output.ptr<float>());
  const int rc =
      kPacked ? sq8_matmul_packed(input.ptr<float>(), weight.ptr<int8_t>(), scale.ptr<float>(), y,
                                  M, N, K, group_size, ws, cfg->workspace_bytes(), cfg->stream)
              : sq8_matmul(input.ptr<float>(), weight.ptr<int8_t>(), scale.ptr<float>(), y, M, N,
                           K, group_size, ws, cfg->workspace_bytes(), cfg->stream);
  CHECK(rc == SQ8_OK) << (kPacked ? "sq8_matmul_packed: " : "sq8_matmul: ")
                      << sq8_status_string(rc);
}
}  // namespace

void matmul_kernel_hip_qint8(const tensor::Tensor& input, const tensor::Tensor& weight,
                             const tensor::Tensor& output, int32_t group_size,
                             const tensor::Tensor& scale, const HipConfig* config) {
  matmul_qint8<false>(input, weight, output, group_size, scale, config);
}

void matmul_kernel_hip_qint8_packed(const tensor::Tensor& input, const tensor::Tensor& weight,
                                    const tensor::Tensor& output, int32_t group_size,
                                    const tensor::Tensor& scale, const HipConfig* config) {
  matmul_qint8<true>(input, weight, output, group_size, scale, config);
}

namespace {
__global__ void add_rows_kernel(const float* a, const float* bias, float* out, size_t n, int K) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    out[i] = a[i] + bias[i % K];
}
}  // namespace

void add_kernel_hip(const tensor::Tensor& input1, const tensor::Tensor& input2,
                    const tensor::Tensor& output, void* stream) {
  CHECK(!input1.is_empty() && !input2.is_empty() && !output.is_empty());
  CHECK_EQ(input1.size(), output.size());
  CHECK_EQ(input1.size() % input2.size(), 0u);
  const size_t n = input1.size();
  const int grid = static_cast<int>(std::min<size_t>((n + 255) / 256, 4096));
  hipLaunchKernelGGL(add_rows_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                     input1.ptr<float>(), input2.ptr<float>(), const_cast<float*>(output.ptr<float>()),
                     n, static_cast<int>(input2.size()));
  CHECK(hipGetLastError() == hipSuccess);
}

MatmulKernelQuant get_matmul_kernel_quant8(base::DeviceType device_type) {
  if (device_type == base::DeviceType::kDeviceHIP) return matmul_kernel_hip_qint8;
  LOG_FATAL << "Unknown device type for get an matmul kernel.";
  return nullptr;
}

MatmulKernelQuant get_matmul_kernel_quant8_packed(base::DeviceType device_type) {
  if (device_type == base::DeviceType::kDeviceHIP) return matmul_kernel_hip_qint8_packed;
  LOG_FATAL << "Unknown device type for get an matmul kernel.";
  return nullptr;
}

AddKernel get_add_kernel(base::DeviceType device_type) {
  if (device_type == base::DeviceType::kDeviceHIP) return add_kernel_hip;
  LOG_FATAL << "Unknown device type for get a add kernel.";
  return nullptr;
}

}  // namespace kernel
