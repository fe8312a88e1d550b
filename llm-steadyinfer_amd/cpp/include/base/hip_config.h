// Per-model device context handed to layers and kernels. Replaces the reference's
// kernel::CudaConfig (src/include/base/cuda_config.h:6-33): a stream plus, here, the device
// workspace the quantised matmul's split-K and activation staging use (the reference kernel needs
// none). The workspace grows on demand and is zero-filled when (re)allocated, as the backend
// requires; grow it before capturing a graph (reserve_workspace).
#ifndef SQ8_OP_BASE_HIP_CONFIG_H_
#define SQ8_OP_BASE_HIP_CONFIG_H_
#include <hip/hip_runtime.h>
#include <cstddef>

namespace kernel {

struct HipConfig {
  hipStream_t stream = nullptr;
  // When true the destructor destroys `stream` (the reference's CudaConfig owns its stream).
  bool owns_stream = false;

  // Returns a device workspace of at least `bytes` (nullptr when bytes == 0). Returns nullptr,
  // allocating nothing, when the workspace would have to grow while `stream` is capturing a
  // graph: reserve_workspace() before the capture.
  void* workspace(size_t bytes);
  size_t workspace_bytes() const { return ws_bytes_; }
  // Grows the workspace now (outside any graph capture).
  void reserve_workspace(size_t bytes) { workspace(bytes); }

  HipConfig() = default;
  HipConfig(const HipConfig&) = delete;
  HipConfig& operator=(const HipConfig&) = delete;
  ~HipConfig();

 private:
  void* ws_ = nullptr;
  size_t ws_bytes_ = 0;
};
using CudaConfig = HipConfig;

}  // namespace kernel
#endif  // SQ8_OP_BASE_HIP_CONFIG_H_
