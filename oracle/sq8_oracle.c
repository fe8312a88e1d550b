/*
 * sq8_oracle.c - CPU restatement of the reference's group-quantised INT8 matmul.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the parity checker and the CPU baseline. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the product library
 * (libsq8.so) never links or calls it.
 *
 * The reference has no CPU INT8 matmul (get_matmul_kernel_quant8 aborts for non-CUDA devices,
 * src/source/op/kernels/kernels_interfaces.cpp:54-61), so the oracle restates:
 *   - the arithmetic of the CUDA kernel matmul_kernel_cu_fp32int8<128>
 *     (src/source/op/kernels/cuda/matmul_kernel.cu:65-99): scale row at scales + (n*K)/gs,
 *     scale of column k at scale_row[k/gs], product x * s * (float)q, fp32 sums;
 *   - the loop structure of the reference CPU fp32 GEMM
 *     (src/source/op/kernels/cpu/matmul_kernel.cpp:55-66): omp parallel over (b, n) rows,
 *     omp simd reduction over k;
 *   - the weight layout of LayerParam::set_weight (src/source/op/layer.cpp:184-218): int8 [N][K]
 *     followed by N*K/gs fp32 scales.
 * Names follow BLAS: M tokens, N outputs, K inputs (the reference calls K "M" and N "K").
 *
 * Parity pins (tests/test_oracle.py): the quantiser against its invariants; sq8o_matmul_f64
 * against numpy's float64 matmul of the dequantised weight and closed-form cases;
 * sq8o_matmul_refgpu_f32 against f64 and against a hand-derived association-order case;
 * sq8o_matmul_cpu_loop against f64. The exact cub BlockReduce bit pattern of the reference GPU
 * kernel cannot be executed here (no CUDA): that bit pattern is "parity unpinned".
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>

/* Group-wise symmetric absmax quantiser defined by the benchmark configs (the reference ships no
 * exporter): groups are consecutive runs of gs elements of the flat N*K array; s = absmax/127 in
 * fp32; q = round-half-away-from-zero(w / s) computed from the fp32 quotient, clamped to +-127;
 * an all-zero group gets s = 0 and q = 0. */
void sq8o_quantize(const float* w, int64_t numel, int gs, int8_t* q, float* s) {
  for (int64_t g0 = 0; g0 < numel; g0 += gs) {
    float amax = 0.f;
    for (int64_t i = g0; i < g0 + gs; ++i) {
      const float a = fabsf(w[i]);
      if (a > amax) amax = a;
    }
    const float sc = amax / 127.0f;
    s[g0 / gs] = sc;
    for (int64_t i = g0; i < g0 + gs; ++i) {
      if (sc == 0.f) {
        q[i] = 0;
        continue;
      }
      const double v = (double)(w[i] / sc);
      double r = floor(fabs(v) + 0.5);
      if (r > 127.0) r = 127.0;
      q[i] = (int8_t)(v < 0 ? -r : r);
    }
  }
}

/* Scale index of (n, k) exactly as the reference computes it (matmul_kernel.cu:77,86). */
static inline int64_t scale_index(int64_t n, int64_t k, int64_t K, int64_t gs) {
  return (n * K) / gs + k / gs;
}

/* Golden: each product x * s * q formed in fp32 as the reference does, accumulated in double. */
void sq8o_matmul_f64(const float* x, const int8_t* w, const float* s, double* y, int M, int N,
                     int K, int gs) {
  for (int m = 0; m < M; ++m) {
    for (int n = 0; n < N; ++n) {
      double acc = 0.0;
      for (int k = 0; k < K; ++k) {
        const float xs = x[(int64_t)m * K + k] * s[scale_index(n, k, K, gs)];
        acc += (double)xs * (double)w[(int64_t)n * K + k];
      }
      y[(int64_t)m * N + n] = acc;
    }
  }
}

/* The reference GPU kernel's fp32 arithmetic and summation order (matmul_kernel.cu:82-97):
 * thread t of 128 accumulates k = t, t+128, ... as fma(x*s, (float)q, acc) (nvcc contracts the
 * multiply-add by default); then cub::BlockReduce<float,128>::Sum with its default
 * warp-reductions algorithm: inside each 32-lane warp a shuffle-down tree with offsets
 * 1, 2, 4, 8, 16 (lane i adds lane i+offset), then warp totals added in warp order. */
void sq8o_matmul_refgpu_f32(const float* x, const int8_t* w, const float* s, float* y, int M,
                            int N, int K, int gs) {
  enum { T = 128, WARP = 32 };
  for (int n = 0; n < N; ++n) {
    for (int m = 0; m < M; ++m) {
      float part[T];
      for (int t = 0; t < T; ++t) {
        float acc = 0.f;
        for (int k = t; k < K; k += T) {
          const float xs = x[(int64_t)m * K + k] * s[scale_index(n, k, K, gs)];
          acc = fmaf(xs, (float)w[(int64_t)n * K + k], acc);
        }
        part[t] = acc;
      }
      float total = 0.f;
      for (int wp = 0; wp < T / WARP; ++wp) {
        float v[WARP];
        for (int l = 0; l < WARP; ++l) v[l] = part[wp * WARP + l];
        for (int off = 1; off < WARP; off <<= 1) {
          float nv[WARP];
          for (int l = 0; l < WARP; ++l) nv[l] = (l + off < WARP) ? v[l] + v[l + off] : v[l];
          for (int l = 0; l < WARP; ++l) v[l] = nv[l];
        }
        total = (wp == 0) ? v[0] : total + v[0];
      }
      y[(int64_t)m * N + n] = total;
    }
  }
}

/* CPU baseline: the reference CPU GEMM loop (cpu/matmul_kernel.cpp:55-66) over the int8 weight,
 * dequantising in the inner loop. Requires K % gs == 0 so that a row's scales are contiguous. */
void sq8o_matmul_cpu_loop(const float* x, const int8_t* w, const float* s, float* y, int M, int N,
                          int K, int gs) {
  const int gpr = K / gs;
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; ++m) {
    for (int n = 0; n < N; ++n) {
      const float* xr = x + (int64_t)m * K;
      const int8_t* wr = w + (int64_t)n * K;
      const float* sr = s + (int64_t)n * gpr;
      float sum = 0.f;
      for (int g = 0; g < gpr; ++g) {
        const float sc = sr[g];
        const int k0 = g * gs;
#pragma omp simd reduction(+ : sum)
        for (int k = k0; k < k0 + gs; ++k) sum += xr[k] * sc * (float)wr[k];
      }
      y[(int64_t)m * N + n] = sum;
    }
  }
}

int sq8o_max_threads(void) {
#ifdef _OPENMP
  extern int omp_get_max_threads(void);
  return omp_get_max_threads();
#else
  return 1;
#endif
}
