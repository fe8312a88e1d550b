// extern "C" boundary of the gfx950 INT8 group-quant matmul backend (declared in include/sq8.h).
//
// Validation mirrors what the reference checks before its launch (matmul_kernel.cu:165-185 and
// layer.cpp:207-211) but reports a status code instead of aborting. Dispatch picks a kernel family
// from the token count M and the alignment of the operands.
#include "../../include/sq8.h"
#include "../../include/sq8_decode.h"
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
  if (!aligned || !fast_shape(K, gs)) return Path::kGeneric;
  if (sq8::gemv_stream_fits(M, K)) return Path::kGemv;
  // The MFMA kernels address weights, scales and activations with 32-bit byte offsets.
  const bool off32 = static_cast<int64_t>(N) * K < (int64_t{1} << 31) &&
                     static_cast<int64_t>(M) * K * 4 < (int64_t{1} << 31);
  if (M >= 3 && gs % 64 == 0 && off32) return Path::kMfma;
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

static size_t align_up(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

// Where an unfused epilogue keeps the product: after the path's own buffers and never in the
// ticket area (a workspace may be shared with MFMA calls whose tickets must stay zero).
static size_t product_offset(size_t base) {
  return align_up(base > sq8::kWsTicketBytes ? base : sq8::kWsTicketBytes);
}

int sq8_epilogue_fused(int M, int N, int K, int group_size) {
  if (M <= 0 || N <= 0 || K <= 0 || group_size <= 0) return 0;
  return choose(M, N, K, group_size, true) == Path::kMfma && sq8::mfma_fuses_epilogue(M, N, K);
}

size_t sq8_epilogue_workspace_bytes(int M, int N, int K, int group_size, int epilogue) {
  const size_t base = sq8_workspace_bytes(M, N, K, group_size);
  if (epilogue == SQ8_EPI_NONE || sq8_epilogue_fused(M, N, K, group_size)) return base;
  return product_offset(base) + static_cast<size_t>(M) * N * sizeof(float);
}

int sq8_matmul_epilogue(const float* x, const int8_t* w, const float* scales, float* y, int M,
                        int N, int K, int group_size, int epilogue, const float* residual,
                        void* workspace, size_t workspace_bytes, void* hip_stream) {
  if (epilogue == SQ8_EPI_NONE)
    return sq8_matmul(x, w, scales, y, M, N, K, group_size, workspace, workspace_bytes,
                      hip_stream);
  if (epilogue != SQ8_EPI_RESIDUAL && epilogue != SQ8_EPI_SWIGLU) return SQ8_ERR_DIMS;
  const int v = validate(x, w, scales, y, M, N, K, group_size);
  if (v != SQ8_OK) return v;
  if (epilogue == SQ8_EPI_RESIDUAL && !residual) return SQ8_ERR_NULL;
  if (epilogue == SQ8_EPI_SWIGLU && N % 2 != 0) return SQ8_ERR_DIMS;
  const size_t need = sq8_epilogue_workspace_bytes(M, N, K, group_size, epilogue);
  if (workspace_bytes < need || (need > 0 && workspace == nullptr)) return SQ8_ERR_WORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(hip_stream);
  const sq8::Epi epi{epilogue, residual};
  const bool aligned = aligned16(x) && aligned16(w);
  hipError_t e;
  if (aligned && sq8_epilogue_fused(M, N, K, group_size)) {
    e = sq8::launch_mfma(x, w, scales, y, M, N, K, group_size, workspace, st, epi);
    return e == hipSuccess ? SQ8_OK : SQ8_ERR_LAUNCH;
  }
  // Unfused: the product goes to the workspace after the path's own buffers.
  const size_t base = sq8_workspace_bytes(M, N, K, group_size);
  float* t = reinterpret_cast<float*>(static_cast<char*>(workspace) + product_offset(base));
  const int r = sq8_matmul(x, w, scales, t, M, N, K, group_size, workspace, base, hip_stream);
  if (r != SQ8_OK) return r;
  e = sq8::launch_epilogue(t, y, M, N, epi, st);
  return e == hipSuccess ? SQ8_OK : SQ8_ERR_LAUNCH;
}

int sq8_rmsnorm_rows_fused(int M, int N, int K, int group_size, int epilogue) {
  if (M <= 0 || N <= 0 || K <= 0 || group_size <= 0) return 0;
  if (epilogue != SQ8_EPI_NONE && epilogue != SQ8_EPI_SWIGLU) return 0;
  if (choose(M, N, K, group_size, true) != Path::kMfma || !sq8::mfma_norm_fused(M, N, K)) return 0;
  return epilogue == SQ8_EPI_NONE || sq8::mfma_fuses_epilogue(M, N, K);
}

size_t sq8_rmsnorm_rows_workspace_bytes(int M, int N, int K, int group_size, int epilogue) {
  if (M <= 0 || N <= 0 || K <= 0 || group_size <= 0) return 0;
  const size_t base = sq8_epilogue_workspace_bytes(M, N, K, group_size, epilogue);
  if (sq8_rmsnorm_rows_fused(M, N, K, group_size, epilogue)) return base;
  // Unfused: the normalised rows follow the matmul's own buffers.
  return product_offset(base) + static_cast<size_t>(M) * K * sizeof(float);
}

int sq8_matmul_rmsnorm_rows(float* x, const float* res, const float* norm_w, float eps,
                            const int8_t* w, const float* scales, float* y, int M, int N, int K,
                            int group_size, int epilogue, void* workspace,
                            size_t workspace_bytes, void* hip_stream) {
  if (!norm_w) return SQ8_ERR_NULL;
  if (epilogue != SQ8_EPI_NONE && epilogue != SQ8_EPI_SWIGLU) return SQ8_ERR_DIMS;
  const int v = validate(x, w, scales, y, M, N, K, group_size);
  if (v != SQ8_OK) return v;
  if (epilogue == SQ8_EPI_SWIGLU && N % 2 != 0) return SQ8_ERR_DIMS;
  const size_t need = sq8_rmsnorm_rows_workspace_bytes(M, N, K, group_size, epilogue);
  if (workspace_bytes < need || (need > 0 && workspace == nullptr)) return SQ8_ERR_WORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(hip_stream);
  const bool aligned = aligned16(x) && aligned16(w) && aligned16(norm_w) &&
                       (!res || aligned16(res));
  if (aligned && sq8_rmsnorm_rows_fused(M, N, K, group_size, epilogue)) {
    const sq8::NormArgs na{x, res, norm_w, eps};
    const hipError_t e = sq8::launch_mfma(x, w, scales, y, M, N, K, group_size, workspace, st,
                                          sq8::Epi{epilogue, nullptr}, &na);
    return e == hipSuccess ? SQ8_OK : SQ8_ERR_LAUNCH;
  }
  // Unfused: the operators' own RMSNorm into the workspace, then the matmul.
  const size_t base = sq8_epilogue_workspace_bytes(M, N, K, group_size, epilogue);
  float* xn = reinterpret_cast<float*>(static_cast<char*>(workspace) + product_offset(base));
  const int r = res ? sq8_add_rmsnorm(x, res, norm_w, xn, M, K, eps, hip_stream)
                    : sq8_rmsnorm(x, norm_w, xn, M, K, eps, hip_stream);
  if (r != SQ8_OK) return r;
  return sq8_matmul_epilogue(xn, w, scales, y, M, N, K, group_size, epilogue, nullptr, workspace,
                             base, hip_stream);
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

// Fused decode projections (include/sq8_decode.h): one token row through the VALU GEMV with its
// input computed while staging. Only shapes that path takes are accepted.
static int validate_fused(const void* x, const void* w, const void* s, const void* y, int N, int K,
                          int gs) {
  if (!x || !w || !s || !y) return SQ8_ERR_NULL;
  if (N <= 0 || K <= 0 || K % 4 != 0 || !sq8::gemv_stream_fits(1, K)) return SQ8_ERR_DIMS;
  if (gs <= 0 || !fast_shape(K, gs)) return SQ8_ERR_GROUP;
  if (!aligned16(x) || !aligned16(w)) return SQ8_ERR_DIMS;
  return SQ8_OK;
}

int sq8_matmul_rmsnorm(const float* x, const float* res, float* x_out, const float* norm_w,
                       float eps, const int8_t* w, const float* scales, float* y, int N, int K,
                       int group_size, void* hip_stream) {
  const int v = validate_fused(x, w, scales, y, N, K, group_size);
  if (v != SQ8_OK) return v;
  if (!norm_w) return SQ8_ERR_NULL;
  if (!aligned16(norm_w) || (res && !aligned16(res)) || (x_out && !aligned16(x_out)))
    return SQ8_ERR_DIMS;
  const hipError_t e = sq8::launch_gemv_norm(x, res, x_out, norm_w, eps, w, scales, y, N, K,
                                             group_size, static_cast<hipStream_t>(hip_stream));
  return e == hipSuccess ? SQ8_OK : SQ8_ERR_LAUNCH;
}

int sq8_matmul_rmsnorm_swiglu(const float* x, const float* res, float* x_out,
                              const float* norm_w, float eps, const int8_t* w,
                              const float* scales, float* y, int N, int K, int group_size,
                              void* hip_stream) {
  const int v = validate_fused(x, w, scales, y, N, K, group_size);
  if (v != SQ8_OK) return v;
  if (!norm_w) return SQ8_ERR_NULL;
  if (N % 2 != 0 || !aligned16(norm_w) || (res && !aligned16(res)) ||
      (x_out && !aligned16(x_out)))
    return SQ8_ERR_DIMS;
  const hipError_t e = sq8::launch_gemv_norm_swiglu(x, res, x_out, norm_w, eps, w, scales, y, N,
                                                    K, group_size,
                                                    static_cast<hipStream_t>(hip_stream));
  return e == hipSuccess ? SQ8_OK : SQ8_ERR_LAUNCH;
}

int sq8_matmul_swiglu(const float* gate_up, const int8_t* w, const float* scales, float* y, int N,
                      int K, int group_size, void* hip_stream) {
  const int v = validate_fused(gate_up, w, scales, y, N, K, group_size);
  if (v != SQ8_OK) return v;
  const hipError_t e = sq8::launch_gemv_swiglu(gate_up, w, scales, y, N, K, group_size,
                                               static_cast<hipStream_t>(hip_stream));
  return e == hipSuccess ? SQ8_OK : SQ8_ERR_LAUNCH;
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
