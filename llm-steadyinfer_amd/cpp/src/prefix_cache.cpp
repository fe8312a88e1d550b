// Prefix cache (src/source/scheduler/prefix_cache.cpp) keyed by whole token prefixes; see
// scheduler/prefix_cache.h for what differs from the reference and why.
#include "scheduler/prefix_cache.h"

#include <algorithm>

namespace scheduler {

// 64-bit FNV-1a over the token ids' bytes, continued from h (chained block by block, so the
// hash of block b covers the whole prefix [0, (b + 1) * block_size)).
uint64_t PrefixCache::chain_hash(uint64_t h, const int* tokens, int n) {
  for (int i = 0; i < n; ++i) {
    uint32_t v = static_cast<uint32_t>(tokens[i]);
    for (int byte = 0; byte < 4; ++byte) {
      h ^= v & 0xffu;
      h *= 1099511628211ull;
      v >>= 8;
    }
  }
  return h;
}

int PrefixCache::shareable_blocks(const std::vector<int>& prompt_tokens) const {
  const int n = static_cast<int>(prompt_tokens.size());
  return n > 0 ? (n - 1) / block_size_ : 0;
}

int PrefixCache::lookup(const std::vector<int>& prompt_tokens, const BlockAllocator& allocator,
                        std::vector<int32_t>* shared_blocks, int max_blocks) const {
  shared_blocks->clear();
  const int nb = std::min(shareable_blocks(prompt_tokens), max_blocks);
  uint64_t h = 14695981039346656037ull;
  for (int b = 0; b < nb; ++b) {
    h = chain_hash(h, prompt_tokens.data() + static_cast<size_t>(b) * block_size_, block_size_);
    const auto it = map_.find(h);
    if (it == map_.end()) break;
    const size_t len = static_cast<size_t>(b + 1) * block_size_;
    int32_t found = -1;
    for (const Entry& e : it->second) {
      const std::vector<int>& owner = *e.owner_prompt;
      if (owner.size() < len || !std::equal(owner.begin(), owner.begin() + len,
                                            prompt_tokens.begin()))
        continue;
      if (allocator.ref_count(e.block_id) > 0 &&
          allocator.allocation_count(e.block_id) == e.allocation &&
          allocator.row_in_use(e.row) &&
          allocator.block_table_row(e.row)[e.block_index] == e.block_id) {
        found = e.block_id;
        break;
      }
    }
    if (found < 0) break;
    shared_blocks->push_back(found);
  }
  return static_cast<int>(shared_blocks->size());
}

void PrefixCache::insert(const std::vector<int>& prompt_tokens, const BlockAllocator& allocator,
                         int row) {
  const int nb = shareable_blocks(prompt_tokens);
  if (nb <= 0) return;
  if (map_.size() >= kMaxEntries) map_.clear();
  auto owner = std::make_shared<const std::vector<int>>(prompt_tokens);
  const int32_t* table = allocator.block_table_row(row);
  uint64_t h = 14695981039346656037ull;
  for (int b = 0; b < nb; ++b) {
    h = chain_hash(h, prompt_tokens.data() + static_cast<size_t>(b) * block_size_, block_size_);
    const int32_t blk = table[b];
    Entry e{row, b, blk, allocator.allocation_count(blk), owner};
    std::vector<Entry>& bucket = map_[h];
    const bool dup = std::any_of(bucket.begin(), bucket.end(), [&](const Entry& o) {
      return o.row == e.row && o.block_index == e.block_index && o.block_id == e.block_id &&
             o.allocation == e.allocation;
    });
    if (!dup) bucket.push_back(std::move(e));
  }
}

}  // namespace scheduler
