// C++ tests of the INT8 model-file loader (model/int8_model_file.h), on files written by
// llm-steadyinfer_amd/model_file.py:
//
//   test_model_file dump <file>     prints the configuration and the byte offset (from the start
//                                   of the weights) of every bound tensor; no GPU calls
//   test_model_file status <file>   prints the status code open() returns; no GPU calls
//   test_model_file gpu <file>      runs projections bound from the file on the device, checked
//                                   against the CPU oracle applied to the mapped bytes
#include <cstdio>
#include <string>
#include <vector>
#include "model/int8_model_file.h"
#include "test_util.h"

extern "C" void sq8o_matmul_f64(const float* x, const int8_t* w, const float* s, double* y, int M,
                                int N, int K, int gs);

namespace {

size_t off(const model::RawModelDataInt8* raw, const void* p) {
  return static_cast<size_t>(static_cast<const int8_t*>(p) -
                             static_cast<const int8_t*>(raw->weight_data));
}

int dump(const std::string& path) {
  model::Int8ModelFile file;
  const base::Status st = file.open(path);
  if (!st) {
    std::printf("open failed: %s\n", st.get_err_msg().c_str());
    return 1;
  }
  model::QuantLayers layers;
  STATUS_CHECK(file.create_quant_layers(base::DeviceType::kDeviceCPU, &layers));
  const auto& c = file.config();
  std::printf("config %d %d %d %d %d %d %d %d %d %d %d %g\n", c.dim_, c.hidden_dim_, c.layer_num_,
              c.head_num_, c.kv_head_num_, c.vocab_size_, c.seq_len_, c.is_shared_weight_ ? 1 : 0,
              file.group_size(), c.kv_dim_, c.head_size_, c.rope_theta_);
  const model::RawModelDataInt8* raw = file.raw();
  auto print = [&](const char* name, const std::vector<std::shared_ptr<op::MatmulLayer>>& v) {
    for (size_t i = 0; i < v.size(); ++i) {
      const auto& w = v[i]->get_weight(0);
      std::printf("quant %s %zu %d %d %zu %zu\n", name, i, w.get_dim(0), w.get_dim(1),
                  off(raw, w.ptr<int8_t>()), off(raw, v[i]->get_scales().ptr<float>()));
    }
  };
  print("wq", layers.wq);
  print("wk", layers.wk);
  print("wv", layers.wv);
  print("wo", layers.wo);
  print("w1", layers.w1);
  print("w2", layers.w2);
  print("w3", layers.w3);
  print("cls", {layers.cls});
  std::printf("fp32 embedding 0 %zu\n", off(raw, layers.embedding));
  for (size_t i = 0; i < layers.rmsnorm.size(); ++i)
    std::printf("fp32 rmsnorm %zu %zu\n", i, off(raw, layers.rmsnorm[i]));
  std::printf("end %zu\n", file.weights_end());
  return 0;
}

void run_layer(const char* name, op::MatmulLayer& layer, int gs, int M) {
  const auto& w = layer.get_weight(0);
  const int N = w.get_dim(0), K = w.get_dim(1);
  // Keep host views of the mapped bytes before to_cuda() moves the layer to the device.
  const int8_t* q = w.ptr<int8_t>();
  const float* s = layer.get_scales().ptr<float>();
  std::vector<double> ref(static_cast<size_t>(M) * N);
  sq8test::Rng r(11 + N + K);
  std::vector<float> x(static_cast<size_t>(M) * K);
  for (auto& v : x) v = r.normal(1.f);
  sq8o_matmul_f64(x.data(), q, s, ref.data(), M, N, K, gs);

  auto cfg = std::make_shared<kernel::HipConfig>();
  CHECK(hipStreamCreate(&cfg->stream) == hipSuccess);
  cfg->owns_stream = true;
  layer.set_cuda_config(cfg);
  layer.to_cuda();
  auto dev = base::HIPDeviceAllocatorFactory::get_instance();
  tensor::Tensor in(base::DataType::kDataTypeFp32, M, K, true, dev);
  tensor::Tensor out(base::DataType::kDataTypeFp32, M, N, true, dev);
  CHECK(hipMemcpy(in.ptr<float>(), x.data(), x.size() * 4, hipMemcpyHostToDevice) == hipSuccess);
  STATUS_CHECK(layer.forward(in, out));
  CHECK(hipStreamSynchronize(cfg->stream) == hipSuccess);
  out.to_cpu();
  std::vector<float> y(out.ptr<float>(), out.ptr<float>() + static_cast<size_t>(M) * N);
  double norm = 0;
  const double elem = sq8test::max_rel_err(y, ref, &norm);
  const bool ok = elem <= 1e-3 && norm <= 1e-5;
  std::printf("%s %s M=%d N=%d K=%d elem=%.2e norm=%.2e\n", ok ? "PASS" : "FAIL", name, M, N, K,
              elem, norm);
  std::fflush(stdout);
  if (!ok) ++sq8test::failures();
}

int gpu(const std::string& path) {
  model::Int8ModelFile file;
  STATUS_CHECK(file.open(path));
  model::QuantLayers layers;
  STATUS_CHECK(file.create_quant_layers(base::DeviceType::kDeviceHIP, &layers));
  const int gs = file.group_size();
  const int L = file.config().layer_num_;
  run_layer("wq[0]", *layers.wq[0], gs, 1);
  run_layer("wk[0]", *layers.wk[0], gs, 3);
  run_layer("w1[last]", *layers.w1[L - 1], gs, 8);
  run_layer("w2[last]", *layers.w2[L - 1], gs, 2);
  if (!file.config().is_shared_weight_) run_layer("cls", *layers.cls, gs, 1);
  std::printf("gpu: %d failure(s)\n", sq8test::failures());
  return sq8test::failures() == 0 ? 0 : 1;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 3) {
    std::printf("usage: %s dump|status|gpu <model file>\n", argv[0]);
    return 2;
  }
  const std::string mode = argv[1], path = argv[2];
  if (mode == "dump") return dump(path);
  if (mode == "status") {
    model::Int8ModelFile file;
    const base::Status st = file.open(path);
    std::printf("status %d\n", st.get_err_code());
    return 0;
  }
  if (mode == "gpu") return gpu(path);
  std::printf("unknown mode %s\n", mode.c_str());
  return 2;
}
