/*
 * sq8_batch.h - C ABI of the continuous-batching operators on gfx950: many token rows from
 * different sequences in one launch, each row at its own position, the KV cache paged.
 *
 * Reference: the batched forward of LLamaModel / Qwen2Model (src/source/model/llama3.cpp:996-1194,
 * forward_batch) driven by the continuous-batching Scheduler (src/source/scheduler/scheduler.cpp).
 * Conventions are those of sq8.h: device pointers owned by the caller, asynchronous on
 * `hip_stream`, nothing allocated, negative status codes on error.
 *
 * Paged KV cache of one layer (one pool for keys, one for values):
 *     cache[block][pos_in_block][kv_dim] fp32, block = block_table[row][pos / block_size],
 *     pos_in_block = pos % block_size
 * (KVManager's paged layout, src/source/scheduler/kv_manager.cpp: [layers, num_blocks, block_size,
 * kv_dim], d innermost). block_table is int32 [rows][table_stride]; positions is int32 [rows].
 */
#ifndef SQ8_BATCH_H_
#define SQ8_BATCH_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* For each row r of qkv (row stride dim + 2*kv_dim: [q | k | v], dim = head_num*head_size,
 * kv_dim = kv_head_num*head_size) at position p = positions[r]: rotates q in place and writes the
 * rotated k and the unchanged v to the row's cache slot for p. Pairs (i, i + head_size/2) of each
 * head rotate by the angle at table column 2i. Replaces rope_kernel_cu_fp32_batch
 * (src/source/op/kernels/cuda/rope_kernel.cu:113-175) followed by paged_kv_scatter_kernel for keys
 * and values (src/source/op/kernels/cuda/paged_kernels.cu:53-90). */
int sq8_paged_rope_kv(float* qkv, int rows, int head_num, int kv_head_num, int head_size,
                      const int32_t* positions, const int32_t* block_table, int table_stride,
                      int block_size, const float* sin_cache, const float* cos_cache,
                      float* key_cache, float* value_cache, void* hip_stream);

/* out[r][h*head_size + d] = attention of query head h of row r (read from qkv with row stride
 * q_stride) over cache positions 0 .. positions[r] of the row's sequence:
 * softmax_t(q . K[t] / sqrt(head_size)) . V[t], kv head h * kv_head_num / head_num.
 * head_size <= 256. Replaces paged_flash_decoding_kernel + its combine
 * (src/source/op/kernels/cuda/paged_kernels.cu:96-294) for decode and prefill rows alike. */
int sq8_paged_attention(const float* qkv, int q_stride, int rows, int head_num, int kv_head_num,
                        int head_size, const int32_t* positions, const int32_t* block_table,
                        int table_stride, int block_size, const float* key_cache,
                        const float* value_cache, float* out, void* hip_stream);

/* sq8_paged_attention with a device workspace that lets long rows split their positions over
 * several workgroups: the flash-decoding split and its combine kernel
 * (src/source/op/kernels/cuda/paged_kernels.cu:96-294), here one launch whose last-finishing
 * chunk per (row, kv head) merges the chunks. The workspace must be zero-filled
 * before its first use (every call leaves it ready for the next); calls that share a workspace
 * must not overlap. workspace == NULL, or a shape for which
 * sq8_paged_attention_workspace_bytes() is 0, runs the unsplit kernel. */
int sq8_paged_attention_ws(const float* qkv, int q_stride, int rows, int head_num,
                           int kv_head_num, int head_size, const int32_t* positions,
                           const int32_t* block_table, int table_stride, int block_size,
                           const float* key_cache, const float* value_cache, float* out,
                           void* workspace, size_t workspace_bytes, void* hip_stream);

/* Workspace bytes sq8_paged_attention_ws uses for any call of at most `rows` rows of this shape
 * (0: it never splits). */
size_t sq8_paged_attention_workspace_bytes(int rows, int head_num, int kv_head_num,
                                           int head_size, int table_stride, int block_size);

/* out[r][i] = silu(gate_up[r][i]) * gate_up[r][ffn + i] for the fused gate/up projection rows
 * [w1 x | w3 x] (swiglu_kernel_cu_fp32, src/source/op/kernels/cuda/swiglu_kernel.cu:4-21, on the
 * separate w1 and w3 outputs). */
int sq8_swiglu_rows(const float* gate_up, int rows, int ffn, float* out, void* hip_stream);

/* out[r] = index of the first maximum of logits[r][0 .. n) (argmax_kernel_batch_fp32,
 * src/source/op/kernels/cuda/argmax_kernel.cu; the single-row sampler uses std::max_element).
 * NaN never wins; an all-NaN row gives 0. */
int sq8_argmax_rows(const float* logits, int rows, int n, int32_t* out, void* hip_stream);

#ifdef __cplusplus
}
#endif

#endif /* SQ8_BATCH_H_ */
