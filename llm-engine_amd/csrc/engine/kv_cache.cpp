// Block allocator and prefix cache. Behaviour of the reference's
// src/kv_cache/block_allocator.cpp (allocation order, refcounts, publication
// only of fully computed blocks, LRU eviction), written for this engine.
#include "kv_cache.h"

#include <cassert>
#include <stdexcept>

namespace le::engine {

namespace {
constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

// splitmix64 finaliser (Steele, Lea, Flood 2014; constants from Vigna's
// public-domain reference implementation).
uint64_t splitmix(uint64_t z) {
  z += kGolden;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
}  // namespace

KVCacheManager::KVCacheManager(int num_blocks, int block_size, bool enable_prefix_caching)
    : num_blocks_(num_blocks), block_size_(block_size), prefix_caching_(enable_prefix_caching) {
  if (num_blocks <= 0 || block_size <= 0)
    throw std::invalid_argument("num_blocks and block_size must be positive");
  refs_.assign(num_blocks, 0);
  hash_of_.assign(num_blocks, 0);
  free_.resize(num_blocks);
  for (int i = 0; i < num_blocks; i++) free_[i] = num_blocks - 1 - i;  // block 0 comes out first
}

uint64_t KVCacheManager::hash_block(uint64_t prev_hash, const int32_t* tokens, int n) {
  uint64_t h = prev_hash ^ kGolden;
  for (int i = 0; i < n; i++) h = splitmix(h ^ static_cast<uint64_t>(static_cast<uint32_t>(tokens[i])));
  return h == 0 ? 1 : h;
}

std::optional<BlockId> KVCacheManager::take_block() {
  if (!free_.empty()) {
    const BlockId b = free_.back();
    free_.pop_back();
    return b;
  }
  if (lru_.empty()) return std::nullopt;
  const BlockId b = lru_.front();  // evict the block released longest ago
  lru_.pop_front();
  lru_at_.erase(b);
  by_hash_.erase(hash_of_[b]);
  hash_of_[b] = 0;
  stats_.evictions++;
  return b;
}

void KVCacheManager::unlink_lru(BlockId b) {
  const auto it = lru_at_.find(b);
  if (it == lru_at_.end()) return;
  lru_.erase(it->second);
  lru_at_.erase(it);
}

void KVCacheManager::release_block(BlockId b, uint64_t hash) {
  assert(refs_[b] > 0);
  if (--refs_[b] > 0) return;
  if (prefix_caching_ && hash != 0 && hash_of_[b] == hash) {
    lru_.push_back(b);  // still a valid prefix block: keep it until evicted
    lru_at_[b] = std::prev(lru_.end());
    return;
  }
  if (hash_of_[b] != 0) {
    by_hash_.erase(hash_of_[b]);
    hash_of_[b] = 0;
  }
  free_.push_back(b);
}

void KVCacheManager::publish(BlockTable& bt, int i, const std::vector<int32_t>& tokens) {
  if (!prefix_caching_) return;
  const uint64_t prev = i == 0 ? 0 : bt.hashes[i - 1];
  if (i > 0 && prev == 0) return;  // the chain broke at an earlier duplicate block
  const uint64_t h = hash_block(prev, tokens.data() + static_cast<size_t>(i) * block_size_, block_size_);
  if (by_hash_.count(h)) return;  // some other block already holds this content
  const BlockId b = bt.blocks[i];
  by_hash_[h] = b;
  hash_of_[b] = h;
  bt.hashes[i] = h;
}

int KVCacheManager::lookup_cached_prefix(const std::vector<int32_t>& tokens) const {
  if (!prefix_caching_) return 0;
  const int full = static_cast<int>(tokens.size()) / block_size_;
  uint64_t prev = 0;
  int hit = 0;
  for (; hit < full; hit++) {
    const uint64_t h = hash_block(prev, tokens.data() + static_cast<size_t>(hit) * block_size_, block_size_);
    if (!by_hash_.count(h)) break;
    prev = h;
  }
  return hit * block_size_;
}

std::optional<int> KVCacheManager::allocate_prompt(BlockTable& bt, const std::vector<int32_t>& tokens) {
  assert(bt.empty());
  const int n = static_cast<int>(tokens.size());
  const int needed = blocks_needed(n, block_size_);
  const int full = n / block_size_;
  stats_.prefix_queries++;
  stats_.prefix_total_blocks += full;

  std::vector<std::pair<uint64_t, BlockId>> hits;
  if (prefix_caching_) {
    uint64_t prev = 0;
    for (int i = 0; i < full; i++) {
      const uint64_t h = hash_block(prev, tokens.data() + static_cast<size_t>(i) * block_size_, block_size_);
      const auto it = by_hash_.find(h);
      if (it == by_hash_.end()) break;
      hits.emplace_back(h, it->second);
      prev = h;
    }
  }
  const int cached = static_cast<int>(hits.size());
  // Cached blocks nobody references sit in the LRU: reusing them does not
  // consume capacity, but they cannot also be counted as allocatable.
  int idle_hits = 0;
  for (const auto& hb : hits) idle_hits += refs_[hb.second] == 0;
  if (needed - cached > num_available_blocks() - idle_hits) {
    stats_.allocation_failures++;
    return std::nullopt;
  }
  for (const auto& hb : hits) {
    unlink_lru(hb.second);
    refs_[hb.second]++;
    bt.blocks.push_back(hb.second);
    bt.hashes.push_back(hb.first);
  }
  stats_.prefix_hit_blocks += cached;
  for (int i = cached; i < needed; i++) {
    const auto b = take_block();
    assert(b.has_value());
    refs_[*b] = 1;
    bt.blocks.push_back(*b);
    bt.hashes.push_back(0);
  }
  bt.num_committed = cached;
  return cached * block_size_;
}

bool KVCacheManager::ensure_slot(BlockTable& bt, int num_tokens) {
  const int needed = blocks_needed(num_tokens, block_size_);
  assert(needed <= bt.num_blocks() + 1);
  if (needed <= bt.num_blocks()) return true;
  const auto b = take_block();
  if (!b) {
    stats_.allocation_failures++;
    return false;
  }
  refs_[*b] = 1;
  bt.blocks.push_back(*b);
  bt.hashes.push_back(0);
  return true;
}

void KVCacheManager::commit_computed(BlockTable& bt, const std::vector<int32_t>& tokens, int num_computed) {
  if (!prefix_caching_) return;
  assert(num_computed <= static_cast<int>(tokens.size()));
  while (bt.num_committed < bt.num_blocks() && (bt.num_committed + 1) * block_size_ <= num_computed) {
    publish(bt, bt.num_committed, tokens);
    bt.num_committed++;
  }
}

void KVCacheManager::free(BlockTable& bt) {
  for (int i = bt.num_blocks() - 1; i >= 0; i--) release_block(bt.blocks[i], bt.hashes[i]);
  bt.blocks.clear();
  bt.hashes.clear();
  bt.num_committed = 0;
}

}  // namespace le::engine
