// Paged KV block pool: the reference's BlockAllocator (src/include/scheduler/block_allocator.h,
// src/source/scheduler/block_allocator.cpp), same interface. One pool serves every layer (block
// i of layer l is kcache[l][i]); one block-table row per running sequence, max_blocks_per_seq
// entries wide, -1 = empty. Blocks carry reference counts so prefix-cache rows can share them
// read-only; a block returns to the LIFO free list when its count reaches zero.
//
// Addition: allocation_count(b) counts how often block b has been handed out. The prefix cache
// records it so that a later allocation of the same block (same row, same index) is never taken
// for the one whose KV it saw.
#ifndef SQ8_OP_SCHEDULER_BLOCK_ALLOCATOR_H_
#define SQ8_OP_SCHEDULER_BLOCK_ALLOCATOR_H_
#include <cstdint>
#include <vector>

namespace scheduler {

class BlockAllocator {
 public:
  BlockAllocator(int num_blocks, int num_rows, int max_blocks_per_seq, int block_size);

  // A free row holding n fresh blocks (n == 0: a row with an empty table); -1 when rows or
  // blocks run out, with nothing changed.
  int allocate_blocks(int n);
  // Mount `blocks` (referenced elsewhere) at the front of `row`, shifting its own blocks right,
  // and take a reference on each. False (nothing changed) when the row is not in use or would
  // overflow.
  bool reserve_shared_prefix(int row, const std::vector<int32_t>& blocks);
  // Release every block of a row and the row itself.
  void free_all(int row);
  // Grow a row by n blocks; the new block count, or -1 with nothing changed.
  int append_blocks(int row, int n);
  // Release entries [start_block_idx, max_blocks_per_seq) of a row (preemption truncation).
  void free_blocks_from(int row, int start_block_idx);
  int num_used_blocks(int row) const;
  void copy_block_table_row(int row, int32_t* dst) const;
  const int32_t* block_table_row(int row) const;
  int free_block_count() const { return static_cast<int>(free_blocks_.size()); }
  bool has_free_blocks(int n) const { return free_block_count() >= n; }
  int num_blocks() const { return num_blocks_; }
  int block_size() const { return block_size_; }
  int max_blocks_per_seq() const { return max_blocks_per_seq_; }
  int num_rows() const { return num_rows_; }
  bool row_in_use(int row) const;

  void inc_ref(int block_idx);
  void dec_ref(int block_idx);
  int ref_count(int block_idx) const;
  uint64_t allocation_count(int block_idx) const;
  // Free list + referenced blocks == num_blocks, every free block unreferenced and listed once.
  bool invariant_holds() const;

 private:
  int take_block();

  int num_blocks_ = 0;
  int num_rows_ = 0;
  int max_blocks_per_seq_ = 0;
  int block_size_ = 0;
  std::vector<int> free_blocks_;       // LIFO: blocks leave as 0, 1, 2, ... from a fresh pool
  std::vector<int> ref_counts_;
  std::vector<uint64_t> alloc_counts_;
  std::vector<int32_t> block_tables_;  // [num_rows][max_blocks_per_seq]
  std::vector<char> row_used_;
};

}  // namespace scheduler
#endif  // SQ8_OP_SCHEDULER_BLOCK_ALLOCATOR_H_
