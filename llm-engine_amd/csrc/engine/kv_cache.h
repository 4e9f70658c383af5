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
  int num_cached_blocks() const { return cached_count_; }
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

  // Test and benchmark aid, not in the reference: reorders the free stack by
  // a seeded Fisher-Yates shuffle (splitmix64 draws), so that allocations
  // hand out a random permutation of the free blocks.
  void shuffle_free_blocks(uint64_t seed);

 private:
  // State of one physical block. A block with no owner but a published hash
  // waits in the reuse queue (an intrusive doubly linked list through
  // `older`/`newer`, oldest release at the head): a later prompt with the same
  // prefix takes it back, memory pressure takes the head first.
  struct Slot {
    int32_t owners = 0;
    uint64_t hash = 0;  // content hash published for this block, 0 if none
    BlockId older = -1, newer = -1;
    bool queued = false;
  };

  // Leading full blocks of `tokens` already published: their ids and hashes
  // (either may be null). Returns how many.
  int walk_prefix(const std::vector<int32_t>& tokens, std::vector<BlockId>* ids,
                  std::vector<uint64_t>* hashes) const;
  BlockId claim();                      // free stack first, else the queue's head; -1 if neither
  void enqueue(BlockId b);              // at the tail (newest)
  void dequeue(BlockId b);
  void forget_hash(BlockId b);
  void drop_owner(BlockId b, uint64_t table_hash);

  int num_blocks_, block_size_;
  bool prefix_caching_;
  std::vector<Slot> slot_;
  std::vector<BlockId> free_;           // a stack: back() is handed out next
  BlockId queue_head_ = -1, queue_tail_ = -1;
  int cached_count_ = 0;
  std::unordered_map<uint64_t, BlockId> published_;
  KVCacheStats stats_;
};

// Bit of a pool-preparation code that selects the shuffled pool; the low 30
// bits are then the seed.
constexpr int kPoolShuffled = 1 << 30;

// Prepares a fresh pool for a run. fragment >= 0 without kPoolShuffled: the
// reference's fragmentation recipe (test_cuda_invariance.cpp:98-105) -
// allocate `fragment` single-block sequences, then free every other one (the
// rest stay allocated; their tables are returned so the caller may keep or
// release them). With kPoolShuffled: the whole free stack in a seeded random
// order, nothing held. Returns the tables still holding blocks.
std::vector<BlockTable> prepare_pool(KVCacheManager& kv, int fragment);

}  // namespace le::engine
