/*
 * sq8_decode.h - C ABI of the single-sequence decode operators around the INT8 matmul on gfx950.
 *
 * These are the layers a decoder step runs between the quantised projections (reference:
 * LLamaModel / Qwen2Model single-token forward, src/source/model/qwen2.cpp:690-830 and
 * src/source/model/llama3.cpp:705-818). Each entry point replaces one reference kernel launcher,
 * cited at its declaration. Conventions are those of sq8.h: device pointers owned by the caller,
 * asynchronous on `hip_stream`, nothing allocated, negative status codes on error.
 *
 * Positions and tokens are read from (and written to) device memory, so a whole decode step can
 * be captured once into a HIP graph and replayed for every token.
 *
 * KV cache layout (one buffer per layer for keys, one for values): [max_seq][kv_dim] fp32, the
 * reference's single-sequence layout (mha_kernel.cu:58, "[num_layers, seq, kv_dim]").
 */
#ifndef SQ8_DECODE_H_
#define SQ8_DECODE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* out[i][:] = table[tokens[i]][:] for i < n; a token outside [0, vocab) leaves its row untouched
 * (emb_kernel_cu_fp32, src/source/op/kernels/cuda/emb_kernel.cu:3-21). */
int sq8_embedding(const float* table, int vocab, int dim, const int32_t* tokens, int n, float* out,
                  void* hip_stream);

/* out[r][:] = rsqrt(mean(x[r][:]^2) + eps) * x[r][:] * w[:] for each of `rows` rows
 * (row_rmsnorm_f32 / row_rmsnorm_f32_dim, src/source/op/kernels/cuda/rmsnorm_kernel.cu:8-160;
 * the reference uses eps = 1e-6). */
int sq8_rmsnorm(const float* x, const float* w, float* out, int rows, int dim, float eps,
                void* hip_stream);

/* Residual add then RMSNorm in one pass: x[r][:] += res[r][:] (written back), then
 * out[r][:] = rmsnorm(x[r][:]) * w. Fuses the reference's VecAddLayer and RmsNormLayer
 * (qwen2.cpp:780-790; add_kernel.cu, rmsnorm_kernel.cu). */
int sq8_add_rmsnorm(float* x, const float* res, const float* w, float* out, int rows, int dim,
                    float eps, void* hip_stream);

/* RoPE tables: sin/cos[pos][j] = sin/cos(pos / theta^(j / head_size)) for pos < max_seq,
 * j < head_size (sin_cos_calc, src/source/op/kernels/cuda/rope_kernel.cu:39-52). */
int sq8_rope_tables(float* sin_cache, float* cos_cache, int head_size, int max_seq, float theta,
                    void* hip_stream);

/* On the fused projection output qkv = [q (dim) | k (kv_dim) | v (kv_dim)] of one token at
 * position *pos: rotates q in place and writes the rotated k and the unchanged v into row *pos of
 * the layer's key and value caches. Pairs (i, i + head_size/2) of each head rotate by the angle
 * at table column 2i (rope_kernel_cu_fp32, rope_kernel.cu:4-37). */
int sq8_rope_kv(float* qkv, int dim, int kv_dim, int head_size, const int32_t* pos,
                const float* sin_cache, const float* cos_cache, float* key_cache,
                float* value_cache, int max_seq, void* hip_stream);

/* Causal attention of one query token at position *pos over cache rows 0..*pos:
 * out[h] = softmax_t(q[h] . K[t][g(h)] / sqrt(head_size)) . V[t][g(h)] with the grouped-query
 * head map g(h) = h * kv_head_num / head_num (flash_decoding_kernel + combine,
 * src/source/op/kernels/cuda/mha_kernel.cu:178-341). head_size <= 256, max_seq <= 2^24; *pos must
 * be below max_seq (the cache rows 0..*pos are read). */
int sq8_attention_decode(const float* q, const float* key_cache, const float* value_cache,
                         const int32_t* pos, float* out, int head_num, int kv_head_num,
                         int head_size, int max_seq, void* hip_stream);

/* sq8_rope_kv followed by sq8_attention_decode in one launch: reads q, k, v from the projection
 * output qkv = [q (head_num*head_size) | k | v] of the token at *pos, rotates q and k, writes the
 * rotated k and v to row *pos of the caches and returns the attention output in out. */
int sq8_rope_attention_decode(const float* qkv, int head_num, int kv_head_num, int head_size,
                              const int32_t* pos, const float* sin_cache, const float* cos_cache,
                              float* key_cache, float* value_cache, float* out, int max_seq,
                              void* hip_stream);

/* sq8_rope_attention_decode with the positions split over several workgroups per head (the
 * flash-decoding split and combine of mha_kernel.cu:178-341, here in one launch: the last chunk
 * of a head to finish merges the chunks). The split is fixed by max_seq (up to 16 chunks of a
 * multiple of 64 positions); chunks past *pos exit at once, and a single live chunk writes its
 * output directly. The workspace (sq8_decode_attention_workspace_bytes; 0: no split for this
 * max_seq) must be zero before its first use and is left ready for the next call; calls that
 * share a workspace must not overlap. workspace == NULL runs the unsplit kernel. */
size_t sq8_decode_attention_workspace_bytes(int head_num, int head_size, int max_seq);
int sq8_rope_attention_decode_ws(const float* qkv, int head_num, int kv_head_num, int head_size,
                                 const int32_t* pos, const float* sin_cache,
                                 const float* cos_cache, float* key_cache, float* value_cache,
                                 float* out, int max_seq, void* workspace, size_t workspace_bytes,
                                 void* hip_stream);

/* out[i] = silu(a[i]) * b[i], silu(v) = v / (1 + exp(-v)) (swiglu_kernel_cu_fp32,
 * src/source/op/kernels/cuda/swiglu_kernel.cu:4-21). `out` may alias `a`. */
int sq8_swiglu(const float* a, const float* b, float* out, int n, void* hip_stream);

/* x[i] += y[i] (add_kernel.cu, used in place as the residual add). */
int sq8_add(float* x, const float* y, int n, void* hip_stream);

/* *out = index of the first maximum of logits[0..n) (ArgmaxSampler::sample,
 * src/source/sampler/argmax_sampler.cpp:5-13: std::max_element). One launch over many
 * workgroups: the workspace (sq8_argmax_workspace_bytes(n)) holds their winners and a ticket; it
 * must be zero before its first use and is left with the ticket zero. Calls that overlap in time
 * on one workspace race. NaN never wins; all-NaN input gives 0. */
size_t sq8_argmax_workspace_bytes(int n);
int sq8_argmax(const float* logits, int n, int32_t* out, void* workspace, size_t workspace_bytes,
               void* hip_stream);

/* The end of a greedy decode step in one launch: *token = first argmax of logits[0..n) (as
 * sq8_argmax, same workspace), *pos += 1, and x[0..dim) = emb_table[*token][0..dim) (the next
 * step's input, emb_kernel_cu_fp32, emb_kernel.cu:3-21; a token outside [0, vocab) leaves x).
 * Replaces the reference's host-side sampler loop (argmax_sampler.cpp:5-13, the position and
 * token update of LLamaModel::predict, llama3.cpp:724) followed by the next step's embedding. */
int sq8_argmax_advance(const float* logits, int n, void* workspace, size_t workspace_bytes,
                       int32_t* pos, int32_t* token, const float* emb_table, int vocab, int dim,
                       float* x, void* hip_stream);

/* Fused decode projections: y[N] = matmul(x', w, scales) for one token row, where x' is formed
 * while the GEMV stages its input (no extra launch, no round trip through memory):
 *   sq8_matmul_rmsnorm: r = x + res (res may be NULL: r = x), x' = rmsnorm(r) * norm_w with the
 *     reference's RMSNorm; r is also written to x_out (may be NULL), which must not alias x or res.
 *     Replaces the reference's add + RMSNorm + projection sequence (qwen2.cpp:780-800).
 *   sq8_matmul_swiglu: gate_up = [a (K) | b (K)], x' = silu(a) * b; replaces SwiGLU + w2
 *     (qwen2.cpp:800-815).
 * The RMSNorm scale rsqrt(mean(r^2) + eps) is applied to the finished dot products (it is one
 * scalar for the row), r * norm_w is what the GEMV stages.
 * Accepted shapes are those of the single-row GEMV: group_size % 16 == 0, K % group_size == 0,
 * 4*K bytes within the 64 KiB activation stage, 16-byte aligned vectors and weights; otherwise
 * SQ8_ERR_DIMS / SQ8_ERR_GROUP. No workspace. */
int sq8_matmul_rmsnorm(const float* x, const float* res, float* x_out, const float* norm_w,
                       float eps, const int8_t* w, const float* scales, float* y, int N, int K,
                       int group_size, void* hip_stream);
int sq8_matmul_swiglu(const float* gate_up, const int8_t* w, const float* scales, float* y, int N,
                      int K, int group_size, void* hip_stream);

/* The FFN input projection of a decode step in one launch: with x' = rmsnorm(x + res) * norm_w
 * as in sq8_matmul_rmsnorm and the fused weight w = [w1; w3] (N = 2F rows, the F gate rows first,
 * each row's scales with it), y[i] = silu(g_i) * u_i for i < F, g = x' . w1^T, u = x' . w3^T:
 * the add, RMSNorm, w1 and w3 projections and SwiGLU of the reference (qwen2.cpp:780-805;
 * swiglu_kernel.cu:4-21). One wave computes both rows of an output. N must be even; other
 * conditions as sq8_matmul_rmsnorm. y holds N/2 values. */
int sq8_matmul_rmsnorm_swiglu(const float* x, const float* res, float* x_out, const float* norm_w,
                              float eps, const int8_t* w, const float* scales, float* y, int N,
                              int K, int group_size, void* hip_stream);

/* Group absmax quantiser on the device, bit-identical to the benchmark quantiser the model files
 * use: per flat group of group_size values s = absmax / 127, q = round-half-away(w / s) clamped
 * to +-127, an all-zero group gives s = 0 and q = 0. numel % group_size must be 0. */
int sq8_quantize(const float* w, int64_t numel, int group_size, int8_t* q, float* scales,
                 void* hip_stream);

/* Decode-loop bookkeeping on the device: *pos += 1 and *token = *next (so a captured step feeds
 * its own output back). No reference counterpart (the reference updates these on the host). */
int sq8_step_advance(int32_t* pos, int32_t* token, const int32_t* next, void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* SQ8_DECODE_H_ */
