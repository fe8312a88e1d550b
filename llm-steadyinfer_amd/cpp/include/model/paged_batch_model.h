// Batched forward over a paged KV cache on gfx950: the reference's LLamaModel::forward_batch and
// decode_step (src/source/model/llama3.cpp:996-1194, model.cpp:74-254) for rows of many
// sequences at their own positions, as scheduler::Scheduler hands them over. Every launch goes
// through the C ABI of libsq8.so (include/sq8.h, sq8_decode.h, sq8_batch.h).
//
// Per step, for the B rows (decode rows first):
//   embedding -> per layer: [add +] RMSNorm -> fused QKV matmul -> paged RoPE + KV write (every
//   row's k, v at its position, before any row attends) -> paged attention (row r over positions
//   0 .. pos[r] of its sequence) -> O matmul -> add + RMSNorm -> fused gate/up matmul + SwiGLU ->
//   down matmul -> add + final RMSNorm -> classifier on the decode rows -> argmax per row.
// The residual add and RMSNorm ahead of QKV and gate/up run inside the matmul's activation
// packing where that kernel fuses them (sq8_matmul_rmsnorm_rows); the residual adds after O and
// down, and the SwiGLU, run in the matmul's output stage where it fuses them
// (sq8_epilogue_fused), else as separate launches.
//
// A decode-only step launches the same kernels for a given B every time, reading tokens,
// positions and block tables from fixed device buffers, so it is captured once per B into a
// HIP graph and replayed (the reference's CUDA-graph decode pool, model.cpp:189-238). Every
// workspace is sized for any B up front, so no step moves a buffer a graph points to, and no
// graph holds a memset (the workspaces are zeroed once, before any capture).
//
// The model does not own its weights: the caller keeps them on the device (row-major, or packed
// by sq8_pack_weights when `packed`) for the model's lifetime. The KV pool is
// [layers][num_blocks][block_size][kv_dim] fp32 for keys and for values (KVManager's paged
// layout, src/source/scheduler/kv_manager.cpp).
#ifndef SQ8_OP_MODEL_PAGED_BATCH_MODEL_H_
#define SQ8_OP_MODEL_PAGED_BATCH_MODEL_H_
#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <vector>

#include "base/base.h"
#include "scheduler/scheduler.h"

namespace model {

struct BatchModelConfig {
  int dim = 0;
  int hidden_dim = 0;  // FFN width
  int layer_num = 0;
  int head_num = 0;
  int kv_head_num = 0;
  int vocab_size = 0;
  float rope_theta = 10000.f;
  int group_size = 64;
  float eps = 1e-6f;
};

// One quantised projection: int8 weight (row-major [N][K] or packed) and its fp32 scales.
struct QuantWeight {
  const int8_t* q = nullptr;
  const float* s = nullptr;
};

struct BatchModelWeights {
  std::vector<QuantWeight> qkv;   // per layer: [wq; wk; wv], (dim + 2 kv_dim) x dim
  std::vector<QuantWeight> o;     // per layer: dim x dim
  std::vector<QuantWeight> gu;    // per layer: [w1; w3], 2 hidden x dim
  std::vector<QuantWeight> down;  // per layer: dim x hidden
  QuantWeight cls;                // vocab x dim
  const float* embedding = nullptr;  // [vocab][dim]
  std::vector<const float*> norm;    // 2 layer_num + 1 vectors of dim: attention norms, FFN
                                     // norms, final norm
  bool packed = false;               // projections in the sq8_pack_weights layout
};

class PagedBatchModel : public scheduler::BatchModel {
 public:
  // stream: the model's stream (nullptr: the model creates one). Call init() before use.
  PagedBatchModel(const BatchModelConfig& cfg, const BatchModelWeights& weights, int max_rows,
                  int max_seq_len, int num_blocks, int block_size, hipStream_t stream = nullptr,
                  bool use_graphs = true, bool split_kv = true);
  ~PagedBatchModel() override;
  PagedBatchModel(const PagedBatchModel&) = delete;
  PagedBatchModel& operator=(const PagedBatchModel&) = delete;

  // Validates the configuration, allocates the KV pool, activations and workspaces and builds
  // the RoPE tables.
  base::Status init();

  base::Status forward_batch(int batch, int num_decode_rows, const int32_t* tokens,
                             const int32_t* positions, const int32_t* seq_ids,
                             const int32_t* block_table, int table_stride,
                             int32_t* next_tokens) override;

  // Captures the decode-only graphs for B = 1 .. max_rows up front, each after one eager run on
  // placeholder rows (token 0 at position 0 of block 0), which writes K/V into block 0 of every
  // layer: an error once forward_batch has run (a sequence may then hold that block). Call it at
  // start-up, as a server does.
  base::Status capture_decode_graphs();

  int64_t graph_replays() const { return graph_replays_; }
  int64_t rows_run() const { return rows_run_; }
  size_t graph_count() const { return graphs_.size(); }
  hipStream_t stream() const { return stream_; }
  int max_blocks_per_seq() const { return max_blocks_per_seq_; }
  size_t kv_pool_bytes() const;

 private:
  base::Status launch(int B, int nd);  // enqueue the forward of the first B staged rows
  base::Status capture(int B);
  base::Status check(int rc, const char* what) const;
  int matmul(const float* x, QuantWeight w, float* y, int M, int N, int K);
  int matmul_epilogue(const float* x, QuantWeight w, float* y, int M, int N, int K, int epi,
                      const float* residual);
  int matmul_norm(float* x, const float* res, const float* norm_w, QuantWeight w, float* y,
                  int M, int N, int K, int epi);

  BatchModelConfig cfg_;
  BatchModelWeights w_;
  int max_rows_, max_seq_len_, num_blocks_, block_size_, max_blocks_per_seq_;
  int head_size_ = 0, kv_dim_ = 0;
  bool use_graphs_, split_kv_;
  hipStream_t stream_ = nullptr;
  bool owns_stream_ = false;
  bool ready_ = false;

  // Device buffers (one allocation each).
  float *kcache_ = nullptr, *vcache_ = nullptr, *sin_ = nullptr, *cos_ = nullptr;
  float *x_ = nullptr, *qkv_ = nullptr, *att_ = nullptr, *proj_ = nullptr, *gu_ = nullptr,
        *hid_ = nullptr, *xn_ = nullptr, *logits_ = nullptr;
  int32_t *tok_d_ = nullptr, *pos_d_ = nullptr, *table_d_ = nullptr, *next_d_ = nullptr;
  void* ws_ = nullptr;
  size_t ws_bytes_ = 0;
  void* att_ws_ = nullptr;
  size_t att_ws_bytes_ = 0;
  // Pinned host staging of the per-step inputs and outputs.
  int32_t *tok_h_ = nullptr, *pos_h_ = nullptr, *table_h_ = nullptr, *next_h_ = nullptr;
  hipEvent_t staged_ = nullptr;  // recorded after each step's uploads from the staging buffers

  std::map<int, hipGraphExec_t> graphs_;
  int64_t graph_replays_ = 0;
  int64_t rows_run_ = 0;
};

}  // namespace model
#endif  // SQ8_OP_MODEL_PAGED_BATCH_MODEL_H_
