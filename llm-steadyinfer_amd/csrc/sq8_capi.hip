// extern "C" boundary of the gfx950 INT8 group-quant matmul backend (declared in include/sq8.h).
//
// Validation mirrors what the reference checks before its launch (matmul_kernel.cu:165-185 and
// layer.cpp:207-211) but reports a status code instead of aborting. Dispatch picks a kernel family
// from the token count M and the alignment of the operands.
#include "../../include/sq8.h"
#include "sq8_common.h"

namespace {

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

enum class Path { kGemv, kMfma, kGeneric };

// Fast kernels need 16-element chunks that never straddle a group and rows that start on a
// group boundary; everything else goes to the exact generic kernel.
bool fast_shape(int K, int gs) { return gs % 16 == 0 && K % gs == 0; }

// Up to 4 token rows whose activations fit the LDS budget go to the VALU GEMV (measured faster
// than the matrix-core kernels there); everything else with 64-wide groups to the MFMA path.
Path choose(int M, int N, int K, int gs, bool aligned) {
  (void)N;
  if (!aligned || !fast_shape(K, gs)) return Path::kGeneric;
  if (sq8::gemv_stream_fits(M, K)) return Path::kGemv;
  if (M >= 3 && gs % 64 == 0) return Path::kMfma;
  return Path::kGemv;
}

int validate(const float* x, const int8_t* w, const float* s, float* y, int M, int N, int K,
             int gs) {
  if (!x || !w || !s || !y) return SQ8_ERR_NULL;
  if (M <= 0 || N <= 0 || K <= 0 || K % 4 != 0) return SQ8_ERR_DIMS;
  if (gs <= 0 || (static_cast<int64_t>(N) * K) % gs != 0) return SQ8_ERR_GROUP;
  return SQ8_OK;
}

}  // namespace

extern "C" {

int sq8_matmul(const float* x, const int8_t* w, const float* scales, float* y, int M, int N, int K,
               int group_size, void* workspace, size_t workspace_bytes, void* hip_stream) {
  const int v = validate(x, w, scales, y, M, N, K, group_size);
  if (v != SQ8_OK) return v;
  const size_t need = sq8_workspace_bytes(M, N, K, group_size);
  if (workspace_bytes < need || (need > 0 && workspace == nullptr)) return SQ8_ERR_WORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(hip_stream);
  const bool aligned = aligned16(x) && aligned16(w);
  hipError_t e = hipSuccess;
  switch (choose(M, N, K, group_size, aligned)) {
    case Path::kGemv:
      e = sq8::launch_gemv(x, w, scales, y, M, N, K, group_size, st);
      break;
    case Path::kMfma:
      e = sq8::launch_mfma(x, w, scales, y, M, N, K, group_size, workspace, st);
      break;
    case Path::kGeneric:
      e = sq8::launch_generic(x, w, scales, y, M, N, K, group_size, st);
      break;
  }
  return e == hipSuccess ? SQ8_OK : SQ8_ERR_LAUNCH;
}

size_t sq8_workspace_bytes(int M, int N, int K, int group_size) {
  if (M <= 0 || N <= 0 || K <= 0 || group_size <= 0) return 0;
  if (choose(M, N, K, group_size, true) != Path::kMfma) return 0;
  return sq8::mfma_workspace_bytes(M, N, K);
}

const char* sq8_status_string(int status) {
  switch (status) {
    case SQ8_OK: return "ok";
    case SQ8_ERR_NULL: return "null pointer argument";
    case SQ8_ERR_DIMS: return "invalid dimensions (M, N, K must be > 0 and K % 4 == 0)";
    case SQ8_ERR_GROUP: return "invalid group size (must be > 0 and divide N*K)";
    case SQ8_ERR_WORKSPACE: return "workspace smaller than sq8_workspace_bytes()";
    case SQ8_ERR_LAUNCH: return "HIP kernel launch failed";
    case SQ8_ERR_DEVICE: return "no usable HIP device";
    default: return "unknown status";
  }
}

const char* sq8_path_name(int M, int N, int K, int group_size) {
  if (M <= 0 || N <= 0 || K <= 0 || group_size <= 0) return "invalid";
  switch (choose(M, N, K, group_size, true)) {
    case Path::kGemv: return "gemv";
    case Path::kMfma: return "mfma";
    case Path::kGeneric: return "generic";
  }
  return "invalid";
}

}  // extern "C"
