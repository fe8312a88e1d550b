/*
 * sq8.h - C ABI of the MI355X (gfx950) group-quantised INT8 matmul backend.
 *
 * The path: y[m, n] = sum_k x[m, k] * scale(n, k) * (float)w[n, k]
 *   x      fp32  [M][K]   activations (M tokens, row-major)
 *   w      int8  [N][K]   symmetric group-quantised weight (row-major, one row per output)
 *   scales fp32  [N*K/group_size]  per-group scales; scale(n, k) = scales[(n*K)/gs + k/gs]
 *   y      fp32  [M][N]   output
 *
 * This replaces the body of the reference's quantised matmul kernel, whose C++ signature is
 *   void matmul_kernel_cu_qint8(const Tensor& input, const Tensor& weight, const Tensor& output,
 *                               int32_t group_size, const Tensor& scale, const CudaConfig* config)
 * (reference: src/source/op/kernels/cuda/matmul_kernel.cu:162-196, typedef MatmulKernelQuant at
 *  src/source/op/kernels/kernels_interface.h:12-14, selected by get_matmul_kernel_quant8 at
 *  src/source/op/kernels/kernels_interfaces.cpp:54-61). The reference names the input width
 *  "M" and the output rows "K" (matmul.cpp:97-100); this header uses BLAS names: M tokens,
 *  N outputs, K inputs.
 *
 * Conventions:
 *   - every pointer is a device pointer owned by the caller; nothing is allocated or freed;
 *   - calls are asynchronous on `hip_stream` (a hipStream_t; NULL = the null stream);
 *   - errors are returned as negative codes (never abort); 0 is success;
 *   - the only global state is a per-device cache of the compute-unit count.
 */
#ifndef SQ8_H_
#define SQ8_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum sq8_status {
  SQ8_OK = 0,
  SQ8_ERR_NULL = -1,        /* a required pointer is NULL */
  SQ8_ERR_DIMS = -2,        /* M, N or K <= 0, or K % 4 != 0 (reference CHECK_EQ(M % 4, 0), matmul_kernel.cu:185) */
  SQ8_ERR_GROUP = -3,       /* group_size <= 0, or N*K not a multiple of group_size (layer.cpp:210) */
  SQ8_ERR_WORKSPACE = -4,   /* workspace smaller than sq8_workspace_bytes() */
  SQ8_ERR_LAUNCH = -5,      /* a HIP launch failed; hipGetLastError() holds the cause */
  SQ8_ERR_DEVICE = -6       /* no usable HIP device */
};

/* Replaces the launch in matmul_kernel_cu_qint8 (matmul_kernel.cu:186-195): computes y for all
 * M token rows of x. Shapes and the scale indexing follow the reference kernel exactly
 * (matmul_kernel.cu:76-88), including group sizes that do not divide K. */
int sq8_matmul(const float* x, const int8_t* w, const float* scales, float* y, int M, int N, int K,
               int group_size, void* workspace, size_t workspace_bytes, void* hip_stream);

/* Bytes of device workspace sq8_matmul needs for this shape (0 when none). The reference
 * kernel needs none (matmul_kernel.cu:65-99); the MFMA paths stage converted activations and
 * split-K partials here. */
size_t sq8_workspace_bytes(int M, int N, int K, int group_size);

/* Packed weights. sq8_pack_weights rewrites a row-major int8 weight [N][K] (K % 64 == 0) into
 * 16-row tiles whose 16 x 64 blocks are stored contiguously, 1 KiB each, in the order the
 * matrix-core kernels load them: byte 16 L + b of block (t, g) is w[16 t + L % 16][64 g +
 * 16 (L / 16) + b]; a tile's K / 64 blocks follow one another, tiles in order, and the rows past N
 * are zero. The scales keep their layout. The reference keeps one row-major layout
 * (layer.cpp:174-231, uploaded by LayerParam::to_cuda); this is an upload-time transform with no
 * reference counterpart, for callers that repack once and keep only the packed copy. Each
 * _packed entry point below computes what its row-major counterpart computes:
 *   - from 3 token rows on, the same kernels with packed addressing: bit-identical results;
 *   - at 1-2 rows (group size 64, K % 256 == 0, 16-byte aligned scales) a packed GEMV whose
 *     summation order differs from the row-major GEMV's (same tolerance to the reference);
 *     other 1-2-row shapes take the int8-limb matrix-core kernel.
 * Requirements: K % 64 == 0, group_size % 64 == 0 and divides K, 16-byte aligned x and packed
 * weights, and a workspace of the _workspace_bytes size (never NULL: the ticket area). */
size_t sq8_packed_weight_bytes(int N, int K);
int sq8_pack_weights(const int8_t* w, int N, int K, int8_t* packed, void* hip_stream);
size_t sq8_packed_workspace_bytes(int M, int N, int K, int group_size);
int sq8_matmul_packed(const float* x, const int8_t* packed, const float* scales, float* y, int M,
                      int N, int K, int group_size, void* workspace, size_t workspace_bytes,
                      void* hip_stream);

/* Output epilogues of sq8_matmul_epilogue. */
enum sq8_epilogue {
  SQ8_EPI_NONE = 0,      /* y[M][N] = x . W^T (as sq8_matmul) */
  SQ8_EPI_RESIDUAL = 1,  /* y[M][N] = residual[M][N] + x . W^T; residual may be y itself */
  SQ8_EPI_SWIGLU = 2     /* W is the fused gate/up weight [w1; w3] (N = 2F rows, the F gate rows
                            first, each row's scales with it); y[M][F] = silu(g) * u with
                            g = x . w1^T, u = x . w3^T, silu(g) = g / (1 + e^-g) */
};

/* y = epilogue(x . W^T) in one pass over the weights where the kernel fuses it. Replaces the
 * separate operators that follow the projections in the reference's batched forward
 * (src/source/model/llama3.cpp:1139-1179): the residual adds after wo and w2
 * (AddLayer, add_kernel.cu) and the SwiGLU of w1/w3 (swiglu_kernel.cu); the reference keeps w1
 * and w3 separate, here they are one fused weight. The prefill GEMM (token counts where
 * sq8_epilogue_fused() is 1) applies the epilogue in its output stage (or in its split-K
 * reduction); other paths run the product into the workspace and apply the epilogue in one
 * elementwise launch. Arguments and errors as sq8_matmul; SQ8_ERR_DIMS if SwiGLU has an odd N,
 * SQ8_ERR_NULL if the residual epilogue has no residual. */
int sq8_matmul_epilogue(const float* x, const int8_t* w, const float* scales, float* y, int M,
                        int N, int K, int group_size, int epilogue, const float* residual,
                        void* workspace, size_t workspace_bytes, void* hip_stream);

/* Workspace bytes of sq8_matmul_epilogue (includes the product buffer of unfused paths). */
size_t sq8_epilogue_workspace_bytes(int M, int N, int K, int group_size, int epilogue);

/* y = epilogue(rmsnorm(x + res) * norm_w . W^T) for M token rows: the reference's residual add
 * and RMSNorm ahead of the QKV and gate/up projections (llama3.cpp:1021-1045, 1139-1150;
 * add_kernel.cu, rmsnorm_kernel.cu:8-160), with x + res written back to x (res may be NULL:
 * x is only read). epilogue is SQ8_EPI_NONE or SQ8_EPI_SWIGLU (y is then [M][N/2]). Where
 * sq8_rmsnorm_rows_fused() is 1 (the MFMA tile and decode-GEMM paths, K <= 16384) the norm is
 * formed while the activation rows are converted for the MFMAs, in the same launch; elsewhere
 * it runs as sq8_add_rmsnorm / sq8_rmsnorm into the workspace, then sq8_matmul_epilogue. */
int sq8_matmul_rmsnorm_rows(float* x, const float* res, const float* norm_w, float eps,
                            const int8_t* w, const float* scales, float* y, int M, int N, int K,
                            int group_size, int epilogue, void* workspace,
                            size_t workspace_bytes, void* hip_stream);
int sq8_rmsnorm_rows_fused(int M, int N, int K, int group_size, int epilogue);
size_t sq8_rmsnorm_rows_workspace_bytes(int M, int N, int K, int group_size, int epilogue);

/* 1 if sq8_matmul_epilogue fuses the epilogue into the matmul kernel for this shape, else 0. */
int sq8_epilogue_fused(int M, int N, int K, int group_size);

/* The epilogue and RMSNorm-rows entry points on packed weights (see sq8_pack_weights above). */
int sq8_epilogue_packed_fused(int M, int N, int K, int group_size);
size_t sq8_epilogue_packed_workspace_bytes(int M, int N, int K, int group_size, int epilogue);
int sq8_matmul_epilogue_packed(const float* x, const int8_t* packed, const float* scales,
                               float* y, int M, int N, int K, int group_size, int epilogue,
                               const float* residual, void* workspace, size_t workspace_bytes,
                               void* hip_stream);
size_t sq8_rmsnorm_rows_packed_workspace_bytes(int M, int N, int K, int group_size,
                                               int epilogue);
int sq8_matmul_rmsnorm_rows_packed(float* x, const float* res, const float* norm_w, float eps,
                                   const int8_t* packed, const float* scales, float* y, int M,
                                   int N, int K, int group_size, int epilogue, void* workspace,
                                   size_t workspace_bytes, void* hip_stream);

/* Size of the device scratch array behind sq8_matmul_noalloc (32 MiB per GPU). */
#define SQ8_NOALLOC_SCRATCH_BYTES (32u * 1024u * 1024u)

/* sq8_matmul without a workspace argument and without any allocation: no counterpart in the
 * reference (whose kernel needs no workspace); for callers that cannot allocate device memory
 * (code under graph capture, tight serving loops, harnesses that forbid hipMalloc). The
 * workspace is a fixed device array of SQ8_NOALLOC_SCRATCH_BYTES in the library, one per GPU,
 * held until the process ends; the first call on a device looks up its address (its split-K
 * tickets start zero and every call leaves them zero, so no call issues a memset or fill, and
 * calls may be captured into a HIP graph and replayed). Shapes whose sq8_workspace_bytes() exceeds it return
 * SQ8_ERR_WORKSPACE (every Llama-3-8B projection up to 64 token rows fits). All calls on one
 * GPU share the array: calls that overlap in time on one GPU (other streams, other threads)
 * race and must not be issued. Results are bitwise those of sq8_matmul. */
int sq8_matmul_noalloc(const float* x, const int8_t* w, const float* scales, float* y, int M,
                       int N, int K, int group_size, void* hip_stream);
size_t sq8_noalloc_scratch_bytes(void);

/* Human-readable text of a status code. */
const char* sq8_status_string(int status);

/* Name of the kernel family sq8_matmul selects for a shape ("gemv", "mfma_skinny",
 * "mfma_gemm", "generic"); lets tests and benchmarks check which path ran. */
const char* sq8_path_name(int M, int N, int K, int group_size);

#ifdef __cplusplus
}
#endif
#endif /* SQ8_H_ */
