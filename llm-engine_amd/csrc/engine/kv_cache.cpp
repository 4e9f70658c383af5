// Block pool and prefix cache of the paged KV cache.
//
// Observable behaviour is the reference KVCacheManager's
// (src/kv_cache/block_allocator.cpp), pinned by the step-by-step block tables
// of the committed scheduler traces:
//   * the pool hands out block 0 first, and a released block is the next one
//     handed out (a stack);
//   * a full block is published under a content hash chained over the blocks
//     before it, only once all its positions are computed, and only if no
//     other block already carries that content (a duplicate ends the chain);
//   * a published block whose last owner releases it is kept for reuse; when
//     the stack is empty the one released longest ago is recycled.
//
// Layout here: one array of per-block records (owner count, published hash,
// links of an intrusive reuse queue), a stack of free ids and one hash index.
// Nothing is allocated per block operation.
#include "kv_cache.h"

#include <algorithm>
#include <stdexcept>

namespace le::engine {

namespace {
constexpr uint64_t kPhi = 0x9E3779B97F4A7C15ull;  // 2^64 / golden ratio

// splitmix64 output function (Steele, Lea and Flood, OOPSLA 2014).
inline uint64_t mix64(uint64_t z) {
  z += kPhi;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
}  // namespace

uint64_t KVCacheManager::hash_block(uint64_t prev_hash, const int32_t* tokens, int n) {
  uint64_t h = prev_hash ^ kPhi;
  for (const int32_t* t = tokens; t != tokens + n; ++t) h = mix64(h ^ static_cast<uint32_t>(*t));
  return h != 0 ? h : 1;  // 0 marks "not published"
}

KVCacheManager::KVCacheManager(int num_blocks, int block_size, bool enable_prefix_caching)
    : num_blocks_(num_blocks), block_size_(block_size), prefix_caching_(enable_prefix_caching) {
  if (num_blocks <= 0 || block_size <= 0)
    throw std::invalid_argument("num_blocks and block_size must be positive");
  slot_.resize(static_cast<size_t>(num_blocks));
  free_.reserve(static_cast<size_t>(num_blocks));
  for (BlockId b = num_blocks; b-- > 0;) free_.push_back(b);
}

void KVCacheManager::shuffle_free_blocks(uint64_t seed) {
  uint64_t state = seed;
  for (size_t i = free_.size(); i > 1; i--) {
    state = mix64(state);
    const size_t j = static_cast<size_t>(state % i);
    std::swap(free_[i - 1], free_[j]);
  }
}

std::vector<BlockTable> prepare_pool(KVCacheManager& kv, int fragment) {
  std::vector<BlockTable> held;
  if (fragment & kPoolShuffled) {
    kv.shuffle_free_blocks(static_cast<uint64_t>(fragment & (kPoolShuffled - 1)));
    return held;
  }
  for (int i = 0; i < fragment; i++) {
    BlockTable bt;
    std::vector<int32_t> one(static_cast<size_t>(std::max(1, kv.block_size() / 2)), 7000 + i);
    if (!kv.allocate_prompt(bt, one)) break;
    held.push_back(bt);
  }
  std::vector<BlockTable> kept;
  for (size_t i = 0; i < held.size(); i++) {
    if (i % 2 == 0) kv.free(held[i]);
    else kept.push_back(held[i]);
  }
  return kept;
}

// ---- reuse queue ----

void KVCacheManager::enqueue(BlockId b) {
  Slot& s = slot_[b];
  s.older = queue_tail_;
  s.newer = -1;
  s.queued = true;
  if (queue_tail_ >= 0) slot_[queue_tail_].newer = b;
  else queue_head_ = b;
  queue_tail_ = b;
  cached_count_++;
}

void KVCacheManager::dequeue(BlockId b) {
  Slot& s = slot_[b];
  if (!s.queued) return;
  (s.older >= 0 ? slot_[s.older].newer : queue_head_) = s.newer;
  (s.newer >= 0 ? slot_[s.newer].older : queue_tail_) = s.older;
  s.older = s.newer = -1;
  s.queued = false;
  cached_count_--;
}

void KVCacheManager::forget_hash(BlockId b) {
  Slot& s = slot_[b];
  if (s.hash == 0) return;
  published_.erase(s.hash);
  s.hash = 0;
}

BlockId KVCacheManager::claim() {
  if (!free_.empty()) {
    const BlockId b = free_.back();
    free_.pop_back();
    return b;
  }
  const BlockId b = queue_head_;
  if (b < 0) return -1;
  dequeue(b);
  forget_hash(b);
  stats_.evictions++;
  return b;
}

// The table recorded `table_hash` for this block when it took it (0 if the
// block was never published through this table). Only a block still carrying
// that hash is worth keeping for reuse.
void KVCacheManager::drop_owner(BlockId b, uint64_t table_hash) {
  Slot& s = slot_[b];
  if (--s.owners > 0) return;
  if (prefix_caching_ && table_hash != 0 && s.hash == table_hash) {
    enqueue(b);
    return;
  }
  forget_hash(b);
  free_.push_back(b);
}

// ---- prefix lookups ----

int KVCacheManager::walk_prefix(const std::vector<int32_t>& tokens, std::vector<BlockId>* ids,
                                std::vector<uint64_t>* hashes) const {
  if (!prefix_caching_) return 0;
  const int full = static_cast<int>(tokens.size()) / block_size_;
  uint64_t chain = 0;
  int n = 0;
  for (; n < full; n++) {
    chain = hash_block(chain, tokens.data() + static_cast<size_t>(n) * block_size_, block_size_);
    const auto hit = published_.find(chain);
    if (hit == published_.end()) break;
    if (ids) ids->push_back(hit->second);
    if (hashes) hashes->push_back(chain);
  }
  return n;
}

int KVCacheManager::lookup_cached_prefix(const std::vector<int32_t>& tokens) const {
  return walk_prefix(tokens, nullptr, nullptr) * block_size_;
}

// ---- sequence operations ----

std::optional<int> KVCacheManager::allocate_prompt(BlockTable& bt, const std::vector<int32_t>& tokens) {
  const int n_tok = static_cast<int>(tokens.size());
  const int want = blocks_needed(n_tok, block_size_);
  stats_.prefix_queries++;
  stats_.prefix_total_blocks += static_cast<uint64_t>(n_tok / block_size_);

  std::vector<BlockId> reuse;
  std::vector<uint64_t> reuse_hash;
  const int hits = walk_prefix(tokens, &reuse, &reuse_hash);
  // A reused block sitting in the queue counts as available, but taking it
  // for this prompt does not free anything: only the rest can come from the
  // pool.
  int queued_hits = 0;
  for (BlockId b : reuse) queued_hits += slot_[b].owners == 0 ? 1 : 0;
  if (want - hits > num_available_blocks() - queued_hits) {
    stats_.allocation_failures++;
    return std::nullopt;
  }

  bt.blocks.assign(reuse.begin(), reuse.end());
  bt.hashes.assign(reuse_hash.begin(), reuse_hash.end());
  for (BlockId b : reuse) {
    dequeue(b);
    slot_[b].owners++;
  }
  while (bt.num_blocks() < want) {
    const BlockId b = claim();  // the capacity check above guarantees one
    slot_[b].owners = 1;
    bt.blocks.push_back(b);
    bt.hashes.push_back(0);
  }
  bt.num_committed = hits;
  stats_.prefix_hit_blocks += static_cast<uint64_t>(hits);
  return hits * block_size_;
}

bool KVCacheManager::ensure_slot(BlockTable& bt, int num_tokens) {
  if (blocks_needed(num_tokens, block_size_) <= bt.num_blocks()) return true;
  const BlockId b = claim();
  if (b < 0) {
    stats_.allocation_failures++;
    return false;
  }
  slot_[b].owners = 1;
  bt.blocks.push_back(b);
  bt.hashes.push_back(0);
  return true;
}

void KVCacheManager::commit_computed(BlockTable& bt, const std::vector<int32_t>& tokens, int num_computed) {
  if (!prefix_caching_) return;
  const int done_blocks = std::min(bt.num_blocks(), num_computed / block_size_);
  for (int i = bt.num_committed; i < done_blocks; i++) {
    bt.num_committed = i + 1;
    // A block whose predecessor was not published (its content already had a
    // block) stays unpublished, and so does everything after it.
    const uint64_t before = i > 0 ? bt.hashes[i - 1] : 0;
    if (i > 0 && before == 0) continue;
    const uint64_t h = hash_block(before, tokens.data() + static_cast<size_t>(i) * block_size_, block_size_);
    const BlockId b = bt.blocks[i];
    if (!published_.emplace(h, b).second) continue;  // another block carries this content
    slot_[b].hash = h;
    bt.hashes[i] = h;
  }
}

void KVCacheManager::free(BlockTable& bt) {
  // Last block first: the first block of the table ends on top of the stack
  // (or newest in the queue).
  for (int i = bt.num_blocks(); i-- > 0;) drop_owner(bt.blocks[i], bt.hashes[i]);
  bt.blocks.clear();
  bt.hashes.clear();
  bt.num_committed = 0;
}

}  // namespace le::engine
