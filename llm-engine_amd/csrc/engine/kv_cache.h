// Paged KV-cache bookkeeping: block tables, refcounted blocks, prefix cache
// with LRU eviction. Pure host logic, no device memory.
//
// Interface and behaviour follow the reference's KVCacheManager
// (include/engine/kv_cache.h:16-99, src/kv_cache/block_allocator.cpp) so a
// scheduler built on it produces the same block tables step for step:
// low block ids are handed out first, a freed block goes back to the top of
// the free list, hashed full blocks of a finished sequence stay cached until
// memory pressure evicts the least recently released one.
#pragma once

#include <cstdint>
#include <list>
#include <optional>
#include <unordered_map>
#include <vector>

namespace le::engine {

using BlockId = int32_t;

struct BlockTable {
  std::vector<BlockId> blocks;
  std::vector<uint64_t> hashes;  // per block; 0 = not published to the prefix cache
  int num_committed = 0;         // leading blocks whose publication was attempted

  int num_blocks() const { return static_cast<int>(blocks.size()); }
  bool empty() const { return blocks.empty(); }
  // Physical slot of logical position `pos` (kv_cache.h:29-31).
  int64_t slot(int pos, int block_size) const {
    return static_cast<int64_t>(blocks[pos / block_size]) * block_size + pos % block_size;
  }
};

struct KVCacheStats {
  uint64_t prefix_queries = 0;
  uint64_t prefix_hit_blocks = 0;
  uint64_t prefix_total_blocks = 0;
  uint64_t evictions = 0;
  uint64_t allocation_failures = 0;
};

class KVCacheManager {
 public:
  KVCacheManager(int num_blocks, int block_size, bool enable_prefix_caching);

  int block_size() const { return block_size_; }
  int num_total_blocks() const { return num_blocks_; }
  int capacity_tokens() const { return num_blocks_ * block_size_; }
  int num_free_blocks() const { return static_cast<int>(free_.size()); }
  int num_cached_blocks() const { return static_cast<int>(lru_.size()); }
  int num_available_blocks() const { return num_free_blocks() + num_cached_blocks(); }
  int num_used_blocks() const { return num_blocks_ - num_available_blocks(); }
  bool prefix_caching_enabled() const { return prefix_caching_; }
  const KVCacheStats& stats() const { return stats_; }

  static int blocks_needed(int num_tokens, int block_size) {
    return (num_tokens + block_size - 1) / block_size;
  }

  // Blocks for a new sequence's prompt. Returns the number of leading prompt
  // tokens already in the cache (a whole number of blocks), or nullopt when
  // the pool cannot hold the prompt now (nothing is allocated then).
  std::optional<int> allocate_prompt(BlockTable& bt, const std::vector<int32_t>& tokens);
  // Makes room for `num_tokens` positions (at most one new block). False when
  // the pool is exhausted.
  bool ensure_slot(BlockTable& bt, int num_tokens);
  // Publishes blocks whose every position is now computed.
  void commit_computed(BlockTable& bt, const std::vector<int32_t>& tokens, int num_computed);
  void free(BlockTable& bt);
  int lookup_cached_prefix(const std::vector<int32_t>& tokens) const;

  // Position-aware content hash of one full block, chained on the previous
  // block's hash (splitmix64 mixing); never 0, which means "unhashed".
  static uint64_t hash_block(uint64_t prev_hash, const int32_t* tokens, int n);

 private:
  std::optional<BlockId> take_block();
  void release_block(BlockId b, uint64_t hash);
  void unlink_lru(BlockId b);
  void publish(BlockTable& bt, int block_idx, const std::vector<int32_t>& tokens);

  int num_blocks_, block_size_;
  bool prefix_caching_;
  std::vector<BlockId> free_;             // back() is handed out next
  std::vector<int> refs_;
  std::vector<uint64_t> hash_of_;         // per physical block, 0 if unpublished
  std::unordered_map<uint64_t, BlockId> by_hash_;
  std::list<BlockId> lru_;                // front = released longest ago
  std::unordered_map<BlockId, std::list<BlockId>::iterator> lru_at_;
  KVCacheStats stats_;
};

}  // namespace le::engine
