// Prefix cache: the reference's PrefixCache (src/include/scheduler/prefix_cache.h,
// src/source/scheduler/prefix_cache.cpp), same interface. A request whose prompt starts with
// whole blocks another sequence has already prefilled mounts those physical blocks read-only
// and skips their prefill. Entries are recorded when the owner's prefill completes and are
// valid only while the block is referenced and still mounted at the recorded (row, index).
//
// Differences, each closing a case where the reference would share KV computed for other
// tokens:
//  - block b is keyed by the whole prefix [0, (b + 1) * block_size): a 64-bit FNV-1a chained
//    over the blocks picks the bucket, and the tokens are compared exactly against the owner's
//    prompt. The reference hashes each block's own tokens only, so a block recorded after a
//    different prefix (different KV) matches, and a hash collision is taken as a match;
//  - an entry also holds the block's allocation count (BlockAllocator::allocation_count): the
//    LIFO free list readily hands a finished owner's block to a new sequence in the same row at
//    the same index, which passes the reference's two checks;
//  - only the blocks before the one holding the prompt's last position are recorded and
//    matched: the scheduler re-runs that position as the sequence's first decode row, so that
//    block is written again and stays private.
#ifndef SQ8_OP_SCHEDULER_PREFIX_CACHE_H_
#define SQ8_OP_SCHEDULER_PREFIX_CACHE_H_
#include <cstddef>
#include <cstdint>
#include <memory>
#include <unordered_map>
#include <vector>

#include "scheduler/block_allocator.h"

namespace scheduler {

class PrefixCache {
 public:
  static constexpr size_t kMaxEntries = size_t{1} << 16;  // then flushed (prefix_cache.cpp:47-53)

  explicit PrefixCache(int block_size) : block_size_(block_size) {}

  // Physical blocks of the longest shareable whole-block prefix, at most max_blocks of them
  // (and never the block of the prompt's last position); returns the count.
  int lookup(const std::vector<int>& prompt_tokens, const BlockAllocator& allocator,
             std::vector<int32_t>* shared_blocks, int max_blocks) const;
  // Record the prompt blocks of `row` before the one holding its last position; call when the
  // sequence's prefill completes.
  void insert(const std::vector<int>& prompt_tokens, const BlockAllocator& allocator, int row);
  size_t entry_count() const { return map_.size(); }

 private:
  struct Entry {
    int row = -1;
    int block_index = 0;
    int32_t block_id = -1;
    uint64_t allocation = 0;
    std::shared_ptr<const std::vector<int>> owner_prompt;  // for the exact prefix comparison
  };
  static uint64_t chain_hash(uint64_t h, const int* tokens, int n);
  int shareable_blocks(const std::vector<int>& prompt_tokens) const;

  int block_size_ = 16;
  std::unordered_map<uint64_t, std::vector<Entry>> map_;
};

}  // namespace scheduler
#endif  // SQ8_OP_SCHEDULER_PREFIX_CACHE_H_
