// The opt-in packed upload of op::MatmulLayer on the host: built with g++ against host stand-ins
// of the HIP runtime and libsq8 (tests/cpp/mock_hip, tests/cpp/mock_sq8.cpp: "device" memory is
// host memory, the repack runs on the host) and a recording kernel table. Checks that
//  * to_cuda() with set_packed_weights(true) keeps one weight tensor, dims [dim0, dim1], whose
//    bytes are the packed layout (checked element by element against the layout's formula:
//    w[n][k] sits at byte 1024 (G (n / 16) + k / 64) + 16 (16 ((k % 64) / 16) + n % 16) + k % 16,
//    rows past N zero);
//  * forward() then calls the packed kernel getter's function with that tensor, and a layer
//    without the opt-in calls the row-major one with its row-major weight;
//  * pack_weights() refuses a host weight, an fp32 layer and a K that is not a multiple of 64.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <vector>

#include "kernels/kernels_interface.h"
#include "op/matmul.h"
#include "test_util.h"

namespace {

struct Seen {
  int rowmajor = 0, packed = 0;
  const void* weight = nullptr;
  int32_t N = 0, K = 0, gs = 0;
} seen;

void record(bool packed, const tensor::Tensor& w, int32_t gs) {
  (packed ? seen.packed : seen.rowmajor) += 1;
  seen.weight = w.ptr<int8_t>();
  seen.N = w.get_dim(0);
  seen.K = w.get_dim(1);
  seen.gs = gs;
}
void rowmajor_kernel(const tensor::Tensor&, const tensor::Tensor& w, const tensor::Tensor&,
                     int32_t gs, const tensor::Tensor&, const kernel::HipConfig*) {
  record(false, w, gs);
}
void packed_kernel(const tensor::Tensor&, const tensor::Tensor& w, const tensor::Tensor&,
                   int32_t gs, const tensor::Tensor&, const kernel::HipConfig*) {
  record(true, w, gs);
}

}  // namespace

namespace kernel {
MatmulKernelQuant get_matmul_kernel_quant8(base::DeviceType) { return rowmajor_kernel; }
MatmulKernelQuant get_matmul_kernel_quant8_packed(base::DeviceType) { return packed_kernel; }
AddKernel get_add_kernel(base::DeviceType) { return nullptr; }
}  // namespace kernel

namespace {

// int8 weights [N][K] then N*K/gs fp32 scales, as LayerParam::set_weight binds them.
std::vector<uint8_t> weight_block(int N, int K, int gs) {
  std::vector<uint8_t> b(static_cast<size_t>(N) * K + static_cast<size_t>(N) * K / gs * 4);
  for (size_t i = 0; i < static_cast<size_t>(N) * K; ++i)
    b[i] = static_cast<uint8_t>((i * 7919u + 13u) % 255u);
  float* s = reinterpret_cast<float*>(b.data() + static_cast<size_t>(N) * K);
  for (size_t i = 0; i < static_cast<size_t>(N) * K / gs; ++i) s[i] = 0.5f + i;
  return b;
}

void run(int N, int K, bool packed) {
  seen = Seen{};
  const int gs = 64;
  auto blob = weight_block(N, K, gs);
  auto cfg = std::make_shared<kernel::HipConfig>();
  op::MatmulLayer layer(base::DeviceType::kDeviceHIP, N, K, true);
  layer.set_group_size(gs);
  EXPECT(layer.set_weight(0, {N, K}, blob.data(), base::DeviceType::kDeviceCPU), "set_weight");
  layer.set_cuda_config(cfg);
  layer.set_packed_weights(packed);
  layer.to_cuda();
  EXPECT(layer.weights_packed() == packed, "weights_packed");
  const tensor::Tensor& w = layer.get_weight(0);
  EXPECT(w.dims_size() == 2 && w.get_dim(0) == N && w.get_dim(1) == K, "dims stay [N, K]");
  EXPECT(w.device_type() == base::DeviceType::kDeviceHIP, "weight on the device");
  const int8_t* d = w.ptr<int8_t>();
  const int G = K / 64, T = (N + 15) / 16;
  long bad = 0;
  if (packed) {
    for (int n = 0; n < T * 16; ++n)
      for (int k = 0; k < K; ++k) {
        const size_t at = 1024 * (static_cast<size_t>(G) * (n / 16) + k / 64) +
                          16 * (16 * ((k % 64) / 16) + n % 16) + k % 16;
        const int8_t want = n < N ? static_cast<int8_t>(blob[static_cast<size_t>(n) * K + k]) : 0;
        bad += d[at] != want;
      }
  } else {
    bad += std::memcmp(d, blob.data(), static_cast<size_t>(N) * K) != 0;
  }
  EXPECT(bad == 0, "uploaded weight bytes");
  // The scales keep their layout.
  const tensor::Tensor& sc = layer.get_scales();
  EXPECT(sc.size() == static_cast<size_t>(N) * K / gs &&
             std::memcmp(sc.ptr<float>(), blob.data() + static_cast<size_t>(N) * K,
                         sc.byte_size()) == 0,
         "scales");

  auto alloc = base::HIPDeviceAllocatorFactory::get_instance();
  tensor::Tensor in(base::DataType::kDataTypeFp32, 3, K, true, alloc);
  tensor::Tensor out(base::DataType::kDataTypeFp32, 3, N, true, alloc);
  EXPECT(layer.forward(in, out), "forward");
  EXPECT(seen.packed == (packed ? 1 : 0) && seen.rowmajor == (packed ? 0 : 1), "kernel choice");
  EXPECT(seen.weight == d && seen.N == N && seen.K == K && seen.gs == gs, "kernel arguments");
  std::printf("%s N=%d K=%d %s\n", sq8test::failures() ? "FAIL" : "PASS", N, K,
              packed ? "packed" : "row-major");
}

}  // namespace

int main() {
  run(40, 128, true);   // a partial last tile (rows 40..47 are padding)
  run(48, 256, true);
  run(40, 128, false);
  {  // refusals, before any repack
    auto blob = weight_block(32, 128, 64);
    op::MatmulLayer host(base::DeviceType::kDeviceHIP, 32, 128, true);
    host.set_group_size(64);
    EXPECT(host.set_weight(0, {32, 128}, blob.data(), base::DeviceType::kDeviceCPU), "bind");
    EXPECT(!host.pack_weights() && !host.weights_packed(), "host weight refused");
    op::MatmulLayer f32(base::DeviceType::kDeviceHIP, 32, 128, false);
    EXPECT(!f32.pack_weights(), "fp32 layer refused");
    auto blob2 = weight_block(16, 96, 32);
    op::MatmulLayer odd(base::DeviceType::kDeviceHIP, 16, 96, true);
    odd.set_group_size(32);
    EXPECT(odd.set_weight(0, {16, 96}, blob2.data(), base::DeviceType::kDeviceCPU), "bind");
    odd.set_cuda_config(std::make_shared<kernel::HipConfig>());
    odd.to_cuda();
    EXPECT(!odd.pack_weights() && !odd.weights_packed(), "K % 64 != 0 refused");
  }
  std::printf("packed layer host: %d failure(s)\n", sq8test::failures());
  return sq8test::failures() == 0 ? 0 : 1;
}
