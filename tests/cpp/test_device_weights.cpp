// Uploads an INT8 model file with model::DeviceWeights, built with g++ against host stand-ins of
// the HIP runtime and libsq8 (tests/cpp/mock_hip, tests/cpp/mock_sq8.cpp: "device" memory is host
// memory and the repack is computed on the host), and writes what it uploaded to a file, in
// order: per layer the QKV, O, gate/up and down weights and scales, then the classifier's, the
// embedding and the 2L + 1 norms. tests/test_native_scheduler.py compares the file with the
// fused layout built in numpy from the same model file.
// usage: test_device_weights <model.bin> <packed 0|1> <out.bin>
#include <cstdio>
#include <cstdlib>

#include "kernels/kernels_interface.h"
#include "model/device_weights.h"

// The op layer's kernel table is not used here (no forward runs).
namespace kernel {
MatmulKernelQuant get_matmul_kernel_quant8(base::DeviceType) { return nullptr; }
MatmulKernelQuant get_matmul_kernel_quant8_packed(base::DeviceType) { return nullptr; }
AddKernel get_add_kernel(base::DeviceType) { return nullptr; }
}  // namespace kernel

void mock_print_log();

int main(int argc, char** argv) {
  if (argc != 4) return 2;
  model::Int8ModelFile f;
  base::Status st = f.open(argv[1]);
  if (!st) {
    std::printf("open failed: %s\n", st.get_err_msg().c_str());
    return 1;
  }
  const bool packed = std::atoi(argv[2]) != 0;
  model::DeviceWeights dw;
  st = dw.upload(f, packed);
  if (!st) {
    std::printf("upload failed: %s\n", st.get_err_msg().c_str());
    return 1;
  }
  const model::BatchModelConfig& c = dw.config();
  const model::BatchModelWeights& w = dw.weights();
  FILE* out = std::fopen(argv[3], "wb");
  if (!out) return 1;
  const int d = c.dim, h = c.hidden_dim, kv = c.kv_head_num * (c.dim / c.head_num);
  auto put = [&](const model::QuantWeight& q, int N, int K) {
    const size_t qb = packed ? static_cast<size_t>((N + 15) / 16) * 16 * K
                             : static_cast<size_t>(N) * K;
    std::fwrite(q.q, 1, qb, out);
    std::fwrite(q.s, sizeof(float), static_cast<size_t>(N) * K / c.group_size, out);
  };
  for (int l = 0; l < c.layer_num; ++l) {
    put(w.qkv[l], d + 2 * kv, d);
    put(w.o[l], d, d);
    put(w.gu[l], 2 * h, d);
    put(w.down[l], d, h);
  }
  put(w.cls, c.vocab_size, d);
  std::fwrite(w.embedding, sizeof(float), static_cast<size_t>(c.vocab_size) * d, out);
  for (const float* n : w.norm) std::fwrite(n, sizeof(float), d, out);
  std::fclose(out);
  std::printf("config %d %d %d %d %d %d %d\n", c.dim, c.hidden_dim, c.layer_num, c.head_num,
              c.kv_head_num, c.vocab_size, c.group_size);
  mock_print_log();
  return 0;
}
