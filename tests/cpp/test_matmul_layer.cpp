// C++ tests of the op API over the gfx950 backend, written the way the reference drives a
// quantised projection: a weight block laid out as in the model file (int8 [N][K] followed by
// fp32 scales, src/source/op/layer.cpp:184-218 and src/source/model/llama3.cpp:193-297), bound with
// set_group_size + set_weight, uploaded with to_cuda, run with forward.
//
//   test_matmul_layer host   host-only checks (no GPU calls)
//   test_matmul_layer gpu    forward on the device, checked against the CPU oracle
//
// The oracle (oracle/_ref/libsq8_oracle.so) is linked as the checker only.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>
#include "kernels/kernels_interface.h"
#include "op/matmul.h"
#include "test_util.h"

extern "C" {
void sq8o_quantize(const float* w, int64_t numel, int gs, int8_t* q, float* s);
void sq8o_matmul_f64(const float* x, const int8_t* w, const float* s, double* y, int M, int N,
                     int K, int gs);
}

namespace {

using sq8test::Rng;
using sq8test::max_rel_err;

// Weight block as the model file stores it: int8 [N][K] then fp32 [N*K/gs] scales.
std::vector<uint8_t> make_weight_block(int N, int K, int gs, uint64_t seed) {
  Rng r(seed);
  std::vector<float> w(static_cast<size_t>(N) * K);
  for (auto& v : w) v = r.normal(0.02f);
  std::vector<uint8_t> blob(w.size() + w.size() / gs * sizeof(float));
  sq8o_quantize(w.data(), static_cast<int64_t>(w.size()), gs, reinterpret_cast<int8_t*>(blob.data()),
                reinterpret_cast<float*>(blob.data() + w.size()));
  return blob;
}

void test_host() {
  const int N = 24, K = 128, gs = 64;
  auto blob = make_weight_block(N, K, gs, 1);
  op::MatmulLayer layer(base::DeviceType::kDeviceCPU, N, K, /*is_quant_layer=*/true);
  layer.set_group_size(gs);
  EXPECT(layer.set_weight(0, {N, K}, blob.data(), base::DeviceType::kDeviceCPU), "set_weight");
  // Scales are read from directly after the int8 block, N*K/gs of them.
  EXPECT(layer.get_scale_num() == N * K / gs, "scale count");
  EXPECT(layer.get_scales().ptr<float>() == reinterpret_cast<const float*>(blob.data() + N * K),
         "scales follow the int8 block");
  EXPECT(layer.get_weight(0).data_type() == base::DataType::kDataTypeInt8, "int8 weight");
  EXPECT(layer.get_weight(0).get_dim(0) == N && layer.get_weight(0).get_dim(1) == K, "dims");

  auto cpu = base::CPUDeviceAllocatorFactory::get_instance();
  tensor::Tensor in(base::DataType::kDataTypeFp32, 3, K, true, cpu);
  tensor::Tensor out(base::DataType::kDataTypeFp32, 3, N, true, cpu);
  layer.set_input(0, in);
  layer.set_output(0, out);
  EXPECT(layer.check(), "valid batched shapes pass check()");
  tensor::Tensor bad_out(base::DataType::kDataTypeFp32, 3, N + 1, true, cpu);
  layer.set_output(0, bad_out);
  EXPECT(layer.check() == base::kInvalidArgument, "wrong output dim is rejected");
  tensor::Tensor in1(base::DataType::kDataTypeFp32, K, true, cpu);
  tensor::Tensor out1(base::DataType::kDataTypeFp32, N, true, cpu);
  layer.set_input(0, in1);
  layer.set_output(0, out1);
  EXPECT(layer.check(), "valid 1-D shapes pass check()");
  tensor::Tensor bad_in(base::DataType::kDataTypeInt32, K, true, cpu);
  layer.set_input(0, bad_in);
  EXPECT(!layer.check(), "wrong input data type is rejected");
  layer.set_input(0, tensor::Tensor());
  EXPECT(!layer.check(), "empty input is rejected");

  op::MatmulLayer bad_group(base::DeviceType::kDeviceCPU, 3, 100, true);
  bad_group.set_group_size(64);  // 300 weights are not a multiple of 64
  auto small = make_weight_block(3, 128, 64, 2);
  EXPECT(bad_group.set_weight(0, {3, 100}, small.data(), base::DeviceType::kDeviceCPU) ==
             base::kInvalidArgument,
         "numel not divisible by the group size");

  tensor::Tensor t(base::DataType::kDataTypeFp32, 2, 3, 4, true, cpu);
  EXPECT(t.size() == 24 && t.byte_size() == 96, "tensor size");
  EXPECT(t.strides() == (std::vector<size_t>{12, 4, 1}), "strides");
  for (int i = 0; i < 24; ++i) t.index<float>(i) = static_cast<float>(i);
  tensor::Tensor c = t.clone();
  c.index<float>(5) = -1.f;
  EXPECT(t.index<float>(5) == 5.f && c.index<float>(23) == 23.f, "clone is a deep copy");
  t.reshape({4, 6});
  EXPECT(t.get_dim(1) == 6 && t.index<float>(7) == 7.f, "reshape keeps data");
  {  // the packed upload refuses what it cannot repack, before any device call
    auto blob = make_weight_block(32, 128, 64, 3);
    op::MatmulLayer q(base::DeviceType::kDeviceHIP, 32, 128, true);
    q.set_group_size(64);
    STATUS_CHECK(q.set_weight(0, {32, 128}, blob.data(), base::DeviceType::kDeviceCPU));
    EXPECT(!q.pack_weights() && !q.weights_packed(), "weight still on the host");
    op::MatmulLayer f(base::DeviceType::kDeviceHIP, 32, 128, false);
    EXPECT(!f.pack_weights(), "fp32 layer");
  }
  std::printf("host checks done\n");
}

std::vector<float> run_case(int M, int N, int K, int gs, bool one_d, bool with_bias,
                            bool packed = false) {
  auto blob = make_weight_block(N, K, gs, 100 + M + N);
  Rng r(7 + M);
  std::vector<float> x(static_cast<size_t>(M) * K);
  for (auto& v : x) v = r.normal(1.f);
  std::vector<float> bias(N);
  for (auto& v : bias) v = r.normal(0.5f);

  auto cfg = std::make_shared<kernel::HipConfig>();
  CHECK(hipStreamCreate(&cfg->stream) == hipSuccess);
  cfg->owns_stream = true;
  op::MatmulLayer layer(base::DeviceType::kDeviceHIP, N, K, true, with_bias);
  layer.set_group_size(gs);
  STATUS_CHECK(layer.set_weight(0, {N, K}, blob.data(), base::DeviceType::kDeviceCPU));
  int32_t nb = N;
  if (with_bias) STATUS_CHECK(layer.set_bias(0, nb, bias.data(), base::DeviceType::kDeviceCPU));
  layer.set_cuda_config(cfg);
  layer.set_packed_weights(packed);
  layer.to_cuda();  // uploads int8 weights, scales and bias (and repacks the weight if asked)
  EXPECT(layer.weights_packed() == packed, "packed upload");

  auto dev = base::HIPDeviceAllocatorFactory::get_instance();
  tensor::Tensor in = one_d ? tensor::Tensor(base::DataType::kDataTypeFp32, K, true, dev)
                            : tensor::Tensor(base::DataType::kDataTypeFp32, M, K, true, dev);
  tensor::Tensor out = one_d ? tensor::Tensor(base::DataType::kDataTypeFp32, N, true, dev)
                             : tensor::Tensor(base::DataType::kDataTypeFp32, M, N, true, dev);
  CHECK(hipMemcpy(in.ptr<float>(), x.data(), x.size() * 4, hipMemcpyHostToDevice) == hipSuccess);
  STATUS_CHECK(layer.forward(in, out));
  CHECK(hipStreamSynchronize(cfg->stream) == hipSuccess);
  out.to_cpu();
  std::vector<float> y(out.ptr<float>(), out.ptr<float>() + static_cast<size_t>(M) * N);

  std::vector<double> ref(static_cast<size_t>(M) * N);
  sq8o_matmul_f64(x.data(), reinterpret_cast<const int8_t*>(blob.data()),
                  reinterpret_cast<const float*>(blob.data() + static_cast<size_t>(N) * K),
                  ref.data(), M, N, K, gs);
  if (with_bias)
    for (int m = 0; m < M; ++m)
      for (int n = 0; n < N; ++n) ref[static_cast<size_t>(m) * N + n] += bias[n];
  double norm = 0;
  const double elem = max_rel_err(y, ref, &norm);
  const bool ok = elem <= 1e-3 && norm <= 1e-5;
  std::printf("%s M=%d N=%d K=%d gs=%d %s%s%s elem=%.2e norm=%.2e\n", ok ? "PASS" : "FAIL", M, N, K,
              gs, one_d ? "1-D" : "2-D", with_bias ? " +bias" : "", packed ? " packed" : "", elem,
              norm);
  std::fflush(stdout);
  if (!ok) ++sq8test::failures();
  return y;
}

// The opt-in packed upload against the row-major one: the oracle's tolerance for both, and
// bit-identical outputs from 3 token rows on (the same kernels with packed addressing).
void run_packed_pair(int M, int N, int K, bool with_bias) {
  const std::vector<float> a = run_case(M, N, K, 64, false, with_bias, false);
  const std::vector<float> b = run_case(M, N, K, 64, false, with_bias, true);
  if (M >= 3) {
    const bool same = a.size() == b.size() &&
                      std::memcmp(a.data(), b.data(), a.size() * sizeof(float)) == 0;
    std::printf("%s packed == row-major bitwise M=%d N=%d K=%d\n", same ? "PASS" : "FAIL", M, N,
                K);
    if (!same) ++sq8test::failures();
  }
}

// A workspace that would have to grow while its stream captures a graph is refused (nullptr, no
// allocation, the old workspace kept); after the capture ends it grows as usual.
void test_workspace_refused_while_capturing() {
  kernel::HipConfig cfg;
  EXPECT(hipStreamCreate(&cfg.stream) == hipSuccess, "stream");
  cfg.owns_stream = true;
  void* small = cfg.workspace(4096);
  EXPECT(small != nullptr && cfg.workspace_bytes() == 4096, "first workspace");
  EXPECT(hipStreamBeginCapture(cfg.stream, hipStreamCaptureModeRelaxed) == hipSuccess,
         "begin capture");
  EXPECT(cfg.workspace(1 << 20) == nullptr, "growth refused while capturing");
  EXPECT(cfg.workspace_bytes() == 4096, "workspace unchanged while capturing");
  EXPECT(cfg.workspace(1024) == small, "a size that fits is served while capturing");
  hipGraph_t graph = nullptr;
  EXPECT(hipStreamEndCapture(cfg.stream, &graph) == hipSuccess, "end capture");
  if (graph) (void)hipGraphDestroy(graph);
  EXPECT(cfg.workspace(1 << 20) != nullptr && cfg.workspace_bytes() == (1u << 20),
         "growth after the capture");
  EXPECT(hipStreamSynchronize(cfg.stream) == hipSuccess, "sync");
}

void test_gpu() {
  run_case(1, 4096, 4096, 64, /*one_d=*/true, false);   // single-token forward() path
  run_case(1, 1000, 1536, 64, false, false);
  run_case(4, 6144, 4096, 64, false, false);
  run_case(16, 512, 14336, 64, false, false);
  run_case(64, 4096, 512, 64, false, false);
  run_case(300, 256, 1024, 64, false, true);            // prefill-sized batch with bias
  run_case(3, 40, 100, 4, false, false);                 // group size the fast kernels cannot take
  // The workspace is reused across layers of different shapes (zero tickets are preserved).
  run_case(8, 4096, 4096, 64, false, false);
  run_case(8, 28672, 4096, 64, false, false);
  // Opt-in packed upload (MatmulLayer::set_packed_weights): the packed GEMV at 1-2 rows, the
  // MFMA kernels with packed addressing from 3 rows on; N not a multiple of 16 pads the last tile.
  run_packed_pair(1, 4096, 4096, false);
  run_packed_pair(2, 1000, 1536, true);
  run_packed_pair(8, 6144, 4096, false);
  run_packed_pair(32, 4104, 4096, false);
  run_packed_pair(300, 256, 1024, true);
  test_workspace_refused_while_capturing();
}

}  // namespace

int main(int argc, char** argv) {
  const std::string mode = argc > 1 ? argv[1] : "host";
  if (mode == "host") {
    test_host();
  } else if (mode == "gpu") {
    test_host();
    test_gpu();
  } else {
    std::printf("usage: %s host|gpu\n", argv[0]);
    return 2;
  }
  std::printf("%s: %d failure(s)\n", mode.c_str(), sq8test::failures());
  return sq8test::failures() == 0 ? 0 : 1;
}
