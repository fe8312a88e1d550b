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

// Weight layouts: row-major [N][K] (the reference's) or packed (sq8_pack_weights).
enum Layout { kRowMajor = 0, kPacked = 1 };

// The packed kernels address weights with 32-bit offsets in the prefill GEMM.
bool packed_shape_ok(int M, int N, int K, int gs) {
  if (M <= 0 || N <= 0 || K <= 0 || gs <= 0) return false;
  if (K % 64 != 0 || gs % 64 != 0 || K % gs != 0) return false;
  return static_cast<int64_t>((N + 15) / 16) * 16 * K < (int64_t{1} << 31) &&
         static_cast<int64_t>(M) * K * 4 < (int64_t{1} << 31);
}

size_t ws_bytes(Layout L, int M, int N, int K, int gs) {
  if (L == kPacked)
    return packed_shape_ok(M, N, K, gs) ? sq8::packed_workspace_bytes(M, N, K, gs) : 0;
  if (M <= 0 || N <= 0 || K <= 0 || gs <= 0) return 0;
  if (choose(M, N, K, gs, true) != Path::kMfma) return 0;
  return sq8::mfma_workspace_bytes(M, N, K);
}

// Packed weights take the MFMA plans from 3 rows on (and the packed GEMV below), so the fused
// epilogue and RMSNorm shapes are the MFMA path's.
bool epi_fused(Layout L, int M, int N, int K, int gs) {
  if (L == kPacked) return packed_shape_ok(M, N, K, gs) && sq8::mfma_fuses_epilogue(M, N, K);
  if (M <= 0 || N <= 0 || K <= 0 || gs <= 0) return false;
  return choose(M, N, K, gs, true) == Path::kMfma && sq8::mfma_fuses_epilogue(M, N, K);
}

size_t align_up(size_t b) { return (b + 255) & ~static_cast<size_t>(255); }

// Where an unfused epilogue keeps the product: after the path's own buffers and never in the
// ticket area (a workspace may be shared with MFMA calls whose tickets must stay zero).
size_t product_offset(size_t base) {
  return align_up(base > sq8::kWsTicketBytes ? base : sq8::kWsTicketBytes);
}

size_t epi_ws_bytes(Layout L, int M, int N, int K, int gs, int epilogue) {
  const size_t base = ws_bytes(L, M, N, K, gs);
  if (epilogue == SQ8_EPI_NONE || epi_fused(L, M, N, K, gs)) return base;
  return product_offset(base) + static_cast<size_t>(M) * N * sizeof(float);
}

int matmul_core(Layout L, const float* x, const int8_t* w, const float* scales, float* y, int M,
                int N, int K, int gs, void* workspace, size_t workspace_bytes, void* hip_stream) {
  const int v = validate(x, w, scales, y, M, N, K, gs);
  if (v != SQ8_OK) return v;
  hipStream_t st = static_cast<hipStream_t>(hip_stream);
  const size_t need = ws_bytes(L, M, N, K, gs);
  if (L == kPacked) {
    if (!packed_shape_ok(M, N, K, gs)) return SQ8_ERR_GROUP;
    if (!aligned16(x) || !aligned16(w)) return SQ8_ERR_DIMS;
    if (workspace_bytes < need || workspace == nullptr) return SQ8_ERR_WORKSPACE;
    const hipError_t e = sq8::launch_mfma(x, w, scales, y, M, N, K, gs, workspace, st,
                                          sq8::Epi{sq8::kEpiNone, nullptr}, nullptr, 1);
    return e == hipSuccess ? SQ8_OK : SQ8_ERR_LAUNCH;
  }
  if (workspace_bytes < need || (need > 0 && workspace == nullptr)) return SQ8_ERR_WORKSPACE;
  const bool aligned = aligned16(x) && aligned16(w);
  hipError_t e = hipSuccess;
  switch (choose(M, N, K, gs, aligned)) {
    case Path::kGemv:
      e = sq8::launch_gemv(x, w, scales, y, M, N, K, gs, st);
      break;
    case Path::kMfma:
      e = sq8::launch_mfma(x, w, scales, y, M, N, K, gs, workspace, st);
      break;
    case Path::kGeneric:
      e = sq8::launch_generic(x, w, scales, y, M, N, K, gs, st);
      break;
  }
  return e == hipSuccess ? SQ8_OK : SQ8_ERR_LAUNCH;
}

int epilogue_core(Layout L, const float* x, const int8_t* w, const float* scales, float* y,
                  int M, int N, int K, int gs, int epilogue, const float* residual,
                  void* workspace, size_t workspace_bytes, void* hip_stream) {
  if (epilogue == SQ8_EPI_NONE)
    return matmul_core(L, x, w, scales, y, M, N, K, gs, workspace, workspace_bytes, hip_stream);
  if (epilogue != SQ8_EPI_RESIDUAL && epilogue != SQ8_EPI_SWIGLU) return SQ8_ERR_DIMS;
  const int v = validate(x, w, scales, y, M, N, K, gs);
  if (v != SQ8_OK) return v;
  if (L == kPacked && !packed_shape_ok(M, N, K, gs)) return SQ8_ERR_GROUP;
  if (epilogue == SQ8_EPI_RESIDUAL && !residual) return SQ8_ERR_NULL;
  if (epilogue == SQ8_EPI_SWIGLU && N % 2 != 0) return SQ8_ERR_DIMS;
  const size_t need = epi_ws_bytes(L, M, N, K, gs, epilogue);
  if (workspace_bytes < need || (need > 0 && workspace == nullptr)) return SQ8_ERR_WORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(hip_stream);
  const sq8::Epi epi{epilogue, residual};
  const bool aligned = aligned16(x) && aligned16(w);
  hipError_t e;
  if (aligned && epi_fused(L, M, N, K, gs)) {
    e = sq8::launch_mfma(x, w, scales, y, M, N, K, gs, workspace, st, epi, nullptr, L);
    return e == hipSuccess ? SQ8_OK : SQ8_ERR_LAUNCH;
  }
  // Unfused: the product goes to the workspace after the path's own buffers.
  const size_t base = ws_bytes(L, M, N, K, gs);
  float* t = reinterpret_cast<float*>(static_cast<char*>(workspace) + product_offset(base));
  const int r = matmul_core(L, x, w, scales, t, M, N, K, gs, workspace, base, hip_stream);
  if (r != SQ8_OK) return r;
  e = sq8::launch_epilogue(t, y, M, N, epi, st);
  return e == hipSuccess ? SQ8_OK : SQ8_ERR_LAUNCH;
}

bool norm_fused(Layout L, int M, int N, int K, int gs, int epilogue) {
  if (M <= 0 || N <= 0 || K <= 0 || gs <= 0) return false;
  if (epilogue != SQ8_EPI_NONE && epilogue != SQ8_EPI_SWIGLU) return false;
  const bool mfma = L == kPacked ? packed_shape_ok(M, N, K, gs)
                                 : choose(M, N, K, gs, true) == Path::kMfma;
  if (!mfma || !sq8::mfma_norm_fused(M, N, K)) return false;
  return epilogue == SQ8_EPI_NONE || sq8::mfma_fuses_epilogue(M, N, K);
}

size_t norm_ws_bytes(Layout L, int M, int N, int K, int gs, int epilogue) {
  if (M <= 0 || N <= 0 || K <= 0 || gs <= 0) return 0;
  const size_t base = epi_ws_bytes(L, M, N, K, gs, epilogue);
  if (norm_fused(L, M, N, K, gs, epilogue)) return base;
  // Unfused: the normalised rows follow the matmul's own buffers.
  return product_offset(base) + static_cast<size_t>(M) * K * sizeof(float);
}

int norm_core(Layout L, float* x, const float* res, const float* norm_w, float eps,
              const int8_t* w, const float* scales, float* y, int M, int N, int K, int gs,
              int epilogue, void* workspace, size_t workspace_bytes, void* hip_stream) {
  if (!norm_w) return SQ8_ERR_NULL;
  if (epilogue != SQ8_EPI_NONE && epilogue != SQ8_EPI_SWIGLU) return SQ8_ERR_DIMS;
  const int v = validate(x, w, scales, y, M, N, K, gs);
  if (v != SQ8_OK) return v;
  if (L == kPacked && !packed_shape_ok(M, N, K, gs)) return SQ8_ERR_GROUP;
  if (epilogue == SQ8_EPI_SWIGLU && N % 2 != 0) return SQ8_ERR_DIMS;
  const size_t need = norm_ws_bytes(L, M, N, K, gs, epilogue);
  if (workspace_bytes < need || (need > 0 && workspace == nullptr)) return SQ8_ERR_WORKSPACE;
  hipStream_t st = static_cast<hipStream_t>(hip_stream);
  const bool aligned = aligned16(x) && aligned16(w) && aligned16(norm_w) &&
                       (!res || aligned16(res));
  if (aligned && norm_fused(L, M, N, K, gs, epilogue)) {
    const sq8::NormArgs na{x, res, norm_w, eps};
    const hipError_t e = sq8::launch_mfma(x, w, scales, y, M, N, K, gs, workspace, st,
                                          sq8::Epi{epilogue, nullptr}, &na, L);
    return e == hipSuccess ? SQ8_OK : SQ8_ERR_LAUNCH;
  }
  // Unfused: the operators' own RMSNorm into the workspace, then the matmul.
  const size_t base = epi_ws_bytes(L, M, N, K, gs, epilogue);
  float* xn = reinterpret_cast<float*>(static_cast<char*>(workspace) + product_offset(base));
  const int r = res ? sq8_add_rmsnorm(x, res, norm_w, xn, M, K, eps, hip_stream)
                    : sq8_rmsnorm(x, norm_w, xn, M, K, eps, hip_stream);
  if (r != SQ8_OK) return r;
  return epilogue_core(L, xn, w, scales, y, M, N, K, gs, epilogue, nullptr, workspace, base,
                       hip_stream);
}

}  // namespace

extern "C" {

int sq8_matmul(const float* x, const int8_t* w, const float* scales, float* y, int M, int N, int K,
               int group_size, void* workspace, size_t workspace_bytes, void* hip_stream) {
  return matmul_core(kRowMajor, x, w, scales, y, M, N, K, group_size, workspace, workspace_bytes,
                     hip_stream);
}

size_t sq8_workspace_bytes(int M, int N, int K, int group_size) {
  return ws_bytes(kRowMajor, M, N, K, group_size);
}

int sq8_epilogue_fused(int M, int N, int K, int group_size) {
  return epi_fused(kRowMajor, M, N, K, group_size);
}

size_t sq8_epilogue_workspace_bytes(int M, int N, int K, int group_size, int epilogue) {
  return epi_ws_bytes(kRowMajor, M, N, K, group_size, epilogue);
}

int sq8_matmul_epilogue(const float* x, const int8_t* w, const float* scales, float* y, int M,
                        int N, int K, int group_size, int epilogue, const float* residual,
                        void* workspace, size_t workspace_bytes, void* hip_stream) {
  return epilogue_core(kRowMajor, x, w, scales, y, M, N, K, group_size, epilogue, residual,
                       workspace, workspace_bytes, hip_stream);
}

int sq8_rmsnorm_rows_fused(int M, int N, int K, int group_size, int epilogue) {
  return norm_fused(kRowMajor, M, N, K, group_size, epilogue);
}

size_t sq8_rmsnorm_rows_workspace_bytes(int M, int N, int K, int group_size, int epilogue) {
  return norm_ws_bytes(kRowMajor, M, N, K, group_size, epilogue);
}

int sq8_matmul_rmsnorm_rows(float* x, const float* res, const float* norm_w, float eps,
                            const int8_t* w, const float* scales, float* y, int M, int N, int K,
                            int group_size, int epilogue, void* workspace,
                            size_t workspace_bytes, void* hip_stream) {
  return norm_core(kRowMajor, x, res, norm_w, eps, w, scales, y, M, N, K, group_size, epilogue,
                   workspace, workspace_bytes, hip_stream);
}

size_t sq8_packed_weight_bytes(int N, int K) {
  if (N <= 0 || K <= 0) return 0;
  return static_cast<size_t>((N + 15) / 16) * 16 * static_cast<size_t>(K);
}

int sq8_pack_weights(const int8_t* w, int N, int K, int8_t* packed, void* hip_stream) {
  if (!w || !packed) return SQ8_ERR_NULL;
  if (N <= 0 || K <= 0 || K % 64 != 0) return SQ8_ERR_DIMS;
  if (!aligned16(w) || !aligned16(packed)) return SQ8_ERR_DIMS;
  const hipError_t e =
      sq8::launch_pack_weights(w, N, K, packed, static_cast<hipStream_t>(hip_stream));
  return e == hipSuccess ? SQ8_OK : SQ8_ERR_LAUNCH;
}

size_t sq8_packed_workspace_bytes(int M, int N, int K, int group_size) {
  return ws_bytes(kPacked, M, N, K, group_size);
}

int sq8_matmul_packed(const float* x, const int8_t* packed, const float* scales, float* y, int M,
                      int N, int K, int group_size, void* workspace, size_t workspace_bytes,
                      void* hip_stream) {
  return matmul_core(kPacked, x, packed, scales, y, M, N, K, group_size, workspace,
                     workspace_bytes, hip_stream);
}

int sq8_epilogue_packed_fused(int M, int N, int K, int group_size) {
  return epi_fused(kPacked, M, N, K, group_size);
}

size_t sq8_epilogue_packed_workspace_bytes(int M, int N, int K, int group_size, int epilogue) {
  return epi_ws_bytes(kPacked, M, N, K, group_size, epilogue);
}

int sq8_matmul_epilogue_packed(const float* x, const int8_t* packed, const float* scales,
                               float* y, int M, int N, int K, int group_size, int epilogue,
                               const float* residual, void* workspace, size_t workspace_bytes,
                               void* hip_stream) {
  return epilogue_core(kPacked, x, packed, scales, y, M, N, K, group_size, epilogue, residual,
                       workspace, workspace_bytes, hip_stream);
}

size_t sq8_rmsnorm_rows_packed_workspace_bytes(int M, int N, int K, int group_size,
                                               int epilogue) {
  return norm_ws_bytes(kPacked, M, N, K, group_size, epilogue);
}

int sq8_matmul_rmsnorm_rows_packed(float* x, const float* res, const float* norm_w, float eps,
                                   const int8_t* packed, const float* scales, float* y, int M,
                                   int N, int K, int group_size, int epilogue, void* workspace,
                                   size_t workspace_bytes, void* hip_stream) {
  return norm_core(kPacked, x, res, norm_w, eps, packed, scales, y, M, N, K, group_size,
                   epilogue, workspace, workspace_bytes, hip_stream);
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
