// Paged KV block pool (src/source/scheduler/block_allocator.cpp): LIFO free list, per-block
// reference counts, one block-table row per running sequence.
#include "scheduler/block_allocator.h"

#include <algorithm>

#include "base/base.h"

namespace scheduler {

BlockAllocator::BlockAllocator(int num_blocks, int num_rows, int max_blocks_per_seq,
                               int block_size)
    : num_blocks_(num_blocks),
      num_rows_(num_rows),
      max_blocks_per_seq_(max_blocks_per_seq),
      block_size_(block_size) {
  CHECK(num_blocks > 0 && num_rows > 0 && max_blocks_per_seq > 0 && block_size > 0)
      << "block pool " << num_blocks << " x " << block_size << ", rows " << num_rows;
  free_blocks_.reserve(num_blocks);
  for (int b = num_blocks - 1; b >= 0; --b) free_blocks_.push_back(b);  // pops give 0, 1, 2, ...
  ref_counts_.assign(num_blocks, 0);
  alloc_counts_.assign(num_blocks, 0);
  block_tables_.assign(static_cast<size_t>(num_rows) * max_blocks_per_seq, -1);
  row_used_.assign(num_rows, 0);
}

int BlockAllocator::take_block() {
  const int b = free_blocks_.back();
  free_blocks_.pop_back();
  CHECK(ref_counts_[b] == 0) << "block " << b << " in the free list with refcount "
                             << ref_counts_[b];
  ref_counts_[b] = 1;
  ++alloc_counts_[b];
  return b;
}

int BlockAllocator::allocate_blocks(int n) {
  if (n < 0 || n > max_blocks_per_seq_ || free_block_count() < n) return -1;
  const auto it = std::find(row_used_.begin(), row_used_.end(), 0);
  if (it == row_used_.end()) return -1;
  const int row = static_cast<int>(it - row_used_.begin());
  row_used_[row] = 1;
  int32_t* t = &block_tables_[static_cast<size_t>(row) * max_blocks_per_seq_];
  for (int i = 0; i < n; ++i) t[i] = take_block();
  return row;
}

bool BlockAllocator::row_in_use(int row) const {
  return row >= 0 && row < num_rows_ && row_used_[row];
}

bool BlockAllocator::reserve_shared_prefix(int row, const std::vector<int32_t>& blocks) {
  if (!row_in_use(row)) return false;
  const int used = num_used_blocks(row);
  const int n = static_cast<int>(blocks.size());
  if (used + n > max_blocks_per_seq_) return false;
  for (int32_t b : blocks)
    if (b < 0 || b >= num_blocks_ || ref_counts_[b] <= 0) return false;
  int32_t* t = &block_tables_[static_cast<size_t>(row) * max_blocks_per_seq_];
  std::copy_backward(t, t + used, t + used + n);  // the row's own blocks move right
  for (int i = 0; i < n; ++i) {
    t[i] = blocks[i];
    ++ref_counts_[blocks[i]];
  }
  return true;
}

int BlockAllocator::append_blocks(int row, int n) {
  if (row < 0 || row >= num_rows_ || n <= 0) return -1;
  const int used = num_used_blocks(row);
  if (used + n > max_blocks_per_seq_ || free_block_count() < n) return -1;
  int32_t* t = &block_tables_[static_cast<size_t>(row) * max_blocks_per_seq_];
  for (int i = 0; i < n; ++i) t[used + i] = take_block();
  return used + n;
}

void BlockAllocator::free_blocks_from(int row, int start_block_idx) {
  if (row < 0 || row >= num_rows_) return;
  int32_t* t = &block_tables_[static_cast<size_t>(row) * max_blocks_per_seq_];
  for (int i = std::max(start_block_idx, 0); i < max_blocks_per_seq_; ++i) {
    const int b = t[i];
    if (b < 0) continue;
    t[i] = -1;
    dec_ref(b);
  }
}

void BlockAllocator::free_all(int row) {
  free_blocks_from(row, 0);
  if (row >= 0 && row < num_rows_) row_used_[row] = 0;
}

int BlockAllocator::num_used_blocks(int row) const {
  if (row < 0 || row >= num_rows_) return 0;
  const int32_t* t = &block_tables_[static_cast<size_t>(row) * max_blocks_per_seq_];
  return static_cast<int>(std::count_if(t, t + max_blocks_per_seq_, [](int32_t b) { return b >= 0; }));
}

void BlockAllocator::copy_block_table_row(int row, int32_t* dst) const {
  CHECK(row >= 0 && row < num_rows_) << "row " << row;
  std::copy_n(block_table_row(row), max_blocks_per_seq_, dst);
}

const int32_t* BlockAllocator::block_table_row(int row) const {
  return &block_tables_[static_cast<size_t>(row) * max_blocks_per_seq_];
}

void BlockAllocator::inc_ref(int block_idx) {
  CHECK(block_idx >= 0 && block_idx < num_blocks_ && ref_counts_[block_idx] > 0)
      << "sharing block " << block_idx;
  ++ref_counts_[block_idx];
}

void BlockAllocator::dec_ref(int block_idx) {
  CHECK(block_idx >= 0 && block_idx < num_blocks_ && ref_counts_[block_idx] > 0)
      << "freeing block " << block_idx;
  if (--ref_counts_[block_idx] == 0) free_blocks_.push_back(block_idx);
}

int BlockAllocator::ref_count(int block_idx) const {
  return block_idx >= 0 && block_idx < num_blocks_ ? ref_counts_[block_idx] : 0;
}

uint64_t BlockAllocator::allocation_count(int block_idx) const {
  return block_idx >= 0 && block_idx < num_blocks_ ? alloc_counts_[block_idx] : 0;
}

bool BlockAllocator::invariant_holds() const {
  std::vector<char> listed(num_blocks_, 0);
  for (int b : free_blocks_) {
    if (b < 0 || b >= num_blocks_ || listed[b] || ref_counts_[b] != 0) return false;
    listed[b] = 1;
  }
  int referenced = 0;
  for (int b = 0; b < num_blocks_; ++b) referenced += ref_counts_[b] > 0;
  return referenced + free_block_count() == num_blocks_;
}

}  // namespace scheduler
