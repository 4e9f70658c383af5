// Ragged step packing (hot-path part 1): le_plan_step / le_plan_upload.
//
// Reference: CudaModel::flatten and upload_step_indices,
// src/model/cuda/cuda_model.cu:434-491, and the CPU twin cpu_model.cpp:107-118.
// The reference builds five int arrays and sends them with six synchronous
// pageable cudaMemcpy calls per step, deduplicating sequences with an O(N*S)
// scan. Here the same arrays (identical values: token ids, positions, int32
// slots, token->sequence index in first-seen order, concatenated tables and
// their offsets) are written into one caller-owned buffer together with
// cu_seqlens_q / seq_lens_k and the attention work lists, then sent with one
// hipMemcpyAsync that every layer of the step shares.
//
// Work lists. A row whose slice has length 1 is a decode row: its context
// 0..pos is cut into partitions of ~partition_tokens (whole blocks, equal
// shares) and each partition becomes one DecodeItem. The rows of a longer
// slice (a prefill chunk) are cut into tiles of chunk_q_tile consecutive
// positions; each tile's keys 0..last position are cut into partitions of
// ~chunk_partition_tokens, one ChunkItem each, run on MFMA tiles (16-bit
// operands with a bf16/fp16 cache, fp32 operands with an fp32 cache). Split
// rows of either kind are merged inside their launch by the last partition
// to finish.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <unordered_map>
#include <vector>

#include "le_internal.h"
#include "llm_engine_amd.h"

namespace {

constexpr int kDefaultPartition = 640;       // decode rows: smallest automatic partition
constexpr int kMaxAutoPartition = 4096;      // decode rows: largest automatic partition
constexpr int kMixedStepPartition = 2048;    // decode rows beside chunk rows: smallest automatic partition
constexpr int kPartitionQuantum = 128;       // 4 waves x 32-key fp32 tiles
constexpr int64_t kTargetItems = 512;        // workgroups per step the sizing aims for (two per CU)
constexpr int kMaxMergeEntries = 1024;       // partitions x group of one decode row (bounds the merge's loads)
constexpr int kDefaultChunkTile = 32;        // query rows per chunk item (two MFMA row tiles)
// Keys per chunk item: one and a half LDS stages. In the one-launch mixed
// step, fewer chunk workgroups leave CUs to the decode rows from the start,
// and fewer partials shorten the tiles' merges (config 3: 256 keys 24.1 us,
// 320 25.1, 384 22.7, 448 23.4, 512 25.0, 768 31.1).
constexpr int kDefaultChunkPartition = 384;
constexpr int kMaxChunkParts = 16;           // partitions of a chunk tile the in-kernel merge stages
constexpr int kMaxChunkItemBlocks = 1024;
constexpr int kXcds = 8;                     // MI355X: XCDs, each with its own L2
constexpr int kItemOverheadBlocks = 8;       // a decode item's fixed cost, in streamed blocks    // block ids of one chunk item the kernel stages

int64_t align256(int64_t x) { return (x + 255) & ~static_cast<int64_t>(255); }

int round_to_blocks(int tokens, int bs) {
  const int b = (tokens + bs - 1) / bs;
  return b < 1 ? 1 : b;
}

// The dispatcher deals a launch's workgroups to the XCDs round robin, so
// workgroups whose linear ids are equal modulo 8 share an XCD, and each XCD
// has its own L2. The partitions of a split chunk tile (always) and of a
// split decode row (LE_PLAN_XCD_LOCAL) are kept on one XCD: the groups (one
// tile's or row's partitions) are dealt longest-first into kXcds bins, each
// to the bin with the least work so far, and item k of bin b goes to index
// k * kXcds + b. Bins are padded to one length with empty items, so the item
// count is a multiple of kXcds and the kv head's offset in the grid (a
// multiple of the item count) keeps every group on its bin's XCD.
template <typename Item, typename Same, typename Blocks>
std::vector<Item> place_on_xcds(const std::vector<Item>& items, Same same_group, Blocks blocks, const Item& pad) {
  struct Group { size_t first, n; int64_t longest, work; };
  std::vector<Group> groups;
  groups.reserve(items.size());
  for (size_t i = 0; i < items.size();) {
    size_t j = i;
    Group g{i, 0, 0, 0};
    while (j < items.size() && same_group(items[j], items[i])) {
      const int64_t nb = blocks(items[j]);
      g.longest = std::max(g.longest, nb);
      g.work += nb + kItemOverheadBlocks;
      j++;
    }
    g.n = j - i;
    groups.push_back(g);
    i = j;
  }
  // longest first; among equally long, the groups with more partitions (the
  // longer merge) first: low ids are dispatched first
  std::stable_sort(groups.begin(), groups.end(), [](const Group& a, const Group& b) {
    return a.longest != b.longest ? a.longest > b.longest : a.n > b.n;
  });
  std::vector<std::vector<Item>> bins(kXcds);
  for (auto& b : bins) b.reserve(items.size() / kXcds + 8);
  int64_t load[kXcds] = {};
  for (const Group& g : groups) {
    int b = 0;
    for (int k = 1; k < kXcds; k++)
      if (load[k] < load[b]) b = k;
    load[b] += g.work;
    for (size_t k = 0; k < g.n; k++) bins[b].push_back(items[g.first + k]);
  }
  size_t len = 0;
  for (const auto& b : bins) len = std::max(len, b.size());
  std::vector<Item> out(len * kXcds, pad);
  for (int b = 0; b < kXcds; b++)
    for (size_t k = 0; k < bins[b].size(); k++) out[k * kXcds + b] = bins[b][k];
  return out;
}

std::vector<le::DecodeItem> place_decode_items(const std::vector<le::DecodeItem>& dec) {
  le::DecodeItem pad{};
  pad.token = -1;
  pad.part = -1;
  pad.n_parts = 0;  // resolved as no work
  return place_on_xcds(
      dec, [](const le::DecodeItem& a, const le::DecodeItem& b) { return a.token == b.token && a.part_begin == b.part_begin; },
      [](const le::DecodeItem& d) { return static_cast<int64_t>(d.blk_end - d.blk_begin); }, pad);
}

std::vector<le::ChunkItem> place_chunk_items(const std::vector<le::ChunkItem>& chk) {
  le::ChunkItem pad{};
  pad.n_q = 0;  // no rows: the workgroup returns at once
  pad.part0 = -1;
  return place_on_xcds(
      chk, [](const le::ChunkItem& a, const le::ChunkItem& b) { return a.tok_begin == b.tok_begin; },
      [](const le::ChunkItem& c) { return static_cast<int64_t>(c.blk_end - c.blk_begin); }, pad);
}

}  // namespace

extern "C" {

int le_plan_step(const le_step_slice* slices, int n_slices, const le_plan_config* cfg_in,
                 void* host_buf, int64_t host_cap, le_step_plan* plan) {
  if (!plan || !cfg_in || n_slices < 0 || (n_slices > 0 && !slices)) return LE_EINVAL;
  le_plan_config cfg = *cfg_in;
  if (cfg.block_size <= 0 || cfg.q_heads <= 0 || cfg.kv_heads <= 0 || cfg.head_dim <= 0)
    return LE_EINVAL;
  if (cfg.kv_dtype != LE_F32 && cfg.kv_dtype != LE_BF16 && cfg.kv_dtype != LE_F16) return LE_EINVAL;
  if ((cfg.flags & ~(LE_PLAN_TWO_LAUNCHES | LE_PLAN_XCD_LOCAL)) != 0 || cfg.table_capacity < 0)
    return LE_EINVAL;
  // Fixed layout (table_capacity > 0): decode rows only, a given partition.
  const bool fixed = cfg.table_capacity > 0;
  if (fixed && cfg.partition_tokens <= 0) return LE_EINVAL;
  const int bs = cfg.block_size;
  if (!fixed && cfg.partition_tokens <= 0) {
    // Size decode partitions so the step has about kTargetItems workgroups,
    // two per CU. Each workgroup pays a fixed chain of dependent memory
    // round trips (block ids, then K/V; partial store, arrival counter, merge)
    // of several microseconds, so on MI355X a few long partitions stream
    // faster than many short ones (measured: 64 x 4096 rows, 2048-token
    // partitions 4.1 TB/s, 256-token 2.2 TB/s; config 2, 640-768 tokens
    // 16.3 us, 1024 17.1 us, 512 18.0 us).
    int64_t ctx = 0;
    for (int i = 0; i < n_slices; i++)
      if (slices[i].len == 1)
        for (int r = 0; r < slices[i].len; r++) ctx += slices[i].start + r + 1;
    const int64_t per_kvh = std::max<int64_t>(1, kTargetItems / cfg.kv_heads);
    int64_t part = (ctx + per_kvh - 1) / per_kvh;
    part = (part + kPartitionQuantum - 1) / kPartitionQuantum * kPartitionQuantum;
    part = std::max<int64_t>(part, kDefaultPartition);
    // In a mixed step the chunk workgroups hold most CUs for the first half
    // of the launch; splitting the decode rows further only adds merges
    // (config 3: 22.7 us with the rule above, 22.4 us with 2048 tokens).
    bool chunk_rows = false;
    for (int i = 0; i < n_slices; i++) chunk_rows |= slices[i].len > 1;
    if (chunk_rows) {
      part = std::max<int64_t>(part, kMixedStepPartition);
    } else {
      // The rows' partitions are whole ceilings, so the rule above can
      // overshoot: grow the partition until the step's workgroups fit one
      // round at two per CU (TinyLlama-shaped decode steps, 64 rows, 4 kv
      // heads: 136-144 items per kv head ran 20.6-21.5 us per launch, 120
      // items 15-16 us).
      const int max_parts = std::max(1, kMaxMergeEntries / std::max(1, cfg.q_heads / cfg.kv_heads));
      auto items_at = [&](int64_t pt) {
        const int64_t pb = (pt + bs - 1) / bs;
        int64_t n = 0;
        for (int i = 0; i < n_slices; i++)
          if (slices[i].len == 1) n += std::min<int64_t>((slices[i].start / bs + 1 + pb - 1) / pb, max_parts);
        return n;
      };
      while (part < kMaxAutoPartition && items_at(part) * cfg.kv_heads > kTargetItems) part += kPartitionQuantum;
    }
    cfg.partition_tokens = static_cast<int32_t>(std::min<int64_t>(part, kMaxAutoPartition));
  }
  if (cfg.chunk_q_tile <= 0) cfg.chunk_q_tile = kDefaultChunkTile;
  // 384 keys: one LDS stage of a 16-bit cache, three of fp32 at head_dim 64
  // (config 3 with fp32 K/V, 24 layers: 1.18 ms per step, against 1.62 with
  // 128-key partitions, 1.47 with 256 and 1.39 with 512)
  if (cfg.chunk_partition_tokens <= 0)
    cfg.chunk_partition_tokens = kDefaultChunkPartition;
  if (cfg.chunk_q_tile != 16 && cfg.chunk_q_tile != 32) return LE_EUNSUPPORTED;  // MFMA row tiles
  const int dec_pb = round_to_blocks(cfg.partition_tokens, bs);
  const int chk_pb = round_to_blocks(cfg.chunk_partition_tokens, bs);
  const bool mfma_chunks = true;  // chunk rows on MFMA tiles, every cache type
  const int max_decode_parts = std::max(1, kMaxMergeEntries / std::max(1, cfg.q_heads / cfg.kv_heads));

  // ---- sizes, and validation of every slice against its table ----
  int64_t n_tok = 0, n_table = 0;
  int n_logits = 0, n_seqs = 0, max_pos = 0;
  std::unordered_map<int64_t, int> seq_index;
  seq_index.reserve(static_cast<size_t>(n_slices));
  std::vector<int> slice_seq(static_cast<size_t>(n_slices));
  std::vector<int> seq_first_slice;
  seq_first_slice.reserve(static_cast<size_t>(n_slices));
  for (int i = 0; i < n_slices; i++) {
    const le_step_slice& s = slices[i];
    if (s.len <= 0 || s.start < 0 || s.num_blocks < 0 || !s.tokens) return LE_EINVAL;
    if (fixed && s.len != 1) return LE_EUNSUPPORTED;
    if (fixed && s.num_blocks > cfg.table_capacity) return LE_EINVAL;
    if (s.num_blocks > 0 && !s.blocks) return LE_EINVAL;
    const int last = s.start + s.len - 1;
    if (last / bs >= s.num_blocks) return LE_EINVAL;  // a position without a block
    auto it = seq_index.find(s.seq_key);
    if (it == seq_index.end()) {
      seq_index.emplace(s.seq_key, n_seqs);
      slice_seq[i] = n_seqs++;
      seq_first_slice.push_back(i);
      n_table += s.num_blocks;
    } else {
      // Slots and block ids come from the sequence's first slice (one table
      // per sequence, as one Sequence object holds it): every later slice of
      // the key must fit that table.
      const le_step_slice& f = slices[seq_first_slice[it->second]];
      if (last / bs >= f.num_blocks) return LE_EINVAL;
      slice_seq[i] = it->second;
    }
    n_tok += s.len;
    if (s.needs_logits) n_logits++;
    max_pos = std::max(max_pos, last);
  }
  if (n_tok > INT32_MAX / 2) return LE_EUNSUPPORTED;
  // Fixed layout: every row owns parts_cap partial slots and every table
  // table_capacity entries, whatever its current length.
  const int parts_cap = fixed ? std::min((cfg.table_capacity + dec_pb - 1) / dec_pb, max_decode_parts) : 0;
  if (fixed) n_table = static_cast<int64_t>(n_seqs) * cfg.table_capacity;

  // Table offset of each distinct sequence in the concatenated tables.
  std::vector<int32_t> seq_table_off(static_cast<size_t>(n_seqs));
  {
    int32_t o = 0;
    for (int s = 0; s < n_seqs; s++) {
      seq_table_off[s] = o;
      o += fixed ? cfg.table_capacity : slices[seq_first_slice[s]].num_blocks;
    }
  }

  // ---- work lists ----
  std::vector<le::DecodeItem> dec;
  std::vector<le::ChunkItem> chk;
  int32_t parts = 0;
  {
    int32_t t = 0;
    for (int i = 0; i < n_slices; i++) {
      const le_step_slice& s = slices[i];
      if (s.len > 1 && mfma_chunks) {
        for (int q0 = 0; q0 < s.len; q0 += cfg.chunk_q_tile) {
          const int nq = std::min(cfg.chunk_q_tile, s.len - q0);
          const int last = s.start + q0 + nq - 1;
          const int nb = last / bs + 1;
          // Long contexts get longer partitions rather than more of them.
          const int pb = std::max(chk_pb, (nb + kMaxChunkParts - 1) / kMaxChunkParts);
          if (pb > kMaxChunkItemBlocks) return LE_EUNSUPPORTED;  // the kernel stages an item's ids in LDS
          const int J = (nb + pb - 1) / pb;
          const int base = J > 1 ? parts : -1;
          for (int j = 0; j < J; j++) {
            le::ChunkItem c{};
            c.tok_begin = t + q0;
            c.n_q = nq;
            c.blk_begin = static_cast<int32_t>(static_cast<int64_t>(j) * nb / J);
            c.blk_end = static_cast<int32_t>(static_cast<int64_t>(j + 1) * nb / J);
            c.part0 = J > 1 ? base + j : -1;
            c.part_stride = J;
            c.seq = slice_seq[i];
            c.part = j;
            c.key_live = std::min((c.blk_end - c.blk_begin) * bs, last + 1 - c.blk_begin * bs);
            chk.push_back(c);
          }
          if (J > 1) parts += nq * J;
        }
      } else {
        for (int r = 0; r < s.len; r++) {
          const int pos = s.start + r;
          const int nb = pos / bs + 1;
          // Partitions per row are capped (the merging workgroup loads them all).
          const int J = std::min((nb + dec_pb - 1) / dec_pb, max_decode_parts);
          // Split rows are merged inside the decode launch by the last
          // partition to finish, so they need no combine item.
          for (int j = 0; j < J; j++) {
            le::DecodeItem d{};
            d.token = t + r;
            d.pos = pos;
            d.table_off = seq_table_off[slice_seq[i]];
            d.blk_begin = static_cast<int32_t>(static_cast<int64_t>(j) * nb / J);
            d.blk_end = static_cast<int32_t>(static_cast<int64_t>(j + 1) * nb / J);
            const int32_t first = fixed ? (t + r) * parts_cap : parts;
            d.part = J > 1 ? first + j : -1;
            d.part_begin = first;
            d.n_parts = J;
            dec.push_back(d);
          }
          if (J > 1 && !fixed) parts += J;
        }
      }
      t += s.len;
    }
  }

  // Longest work first: workgroups start over a couple of microseconds in
  // launch order, so the items on the critical path (most keys) go first.
  // Merges do not depend on the order (partials are addressed by index).
  if (fixed) parts = static_cast<int32_t>(n_tok) * parts_cap;
  // (With the XCD placement, the bins are dealt longest group first instead:
  // a row's partitions must stay adjacent until they are placed.)
  const bool xcd_local = (cfg.flags & LE_PLAN_XCD_LOCAL) && !fixed;
  bool dec_split = false;
  for (const auto& d : dec) dec_split |= d.part >= 0;
  if (xcd_local && dec_split) {
    dec = place_decode_items(dec);
  } else {
    std::stable_sort(dec.begin(), dec.end(), [](const le::DecodeItem& a, const le::DecodeItem& b) {
      return a.blk_end - a.blk_begin > b.blk_end - b.blk_begin;
    });
  }
  bool chunk_split = false;
  for (const auto& c : chk) chunk_split |= c.part0 >= 0;
  if (chunk_split) {
    chk = place_chunk_items(chk);
  } else {
    std::stable_sort(chk.begin(), chk.end(), [](const le::ChunkItem& a, const le::ChunkItem& b) {
      return a.blk_end - a.blk_begin > b.blk_end - b.blk_begin;
    });
  }

  if (fixed) {
    // one item count for every step of this row count: each row has at most
    // parts_cap partitions, so rows * parts_cap items, padded with empty
    // ones (n_parts 0: resolved as no work)
    const size_t cap_items = static_cast<size_t>(n_tok) * parts_cap;
    if (dec.size() > cap_items) return LE_EUNSUPPORTED;  // unreachable: J <= parts_cap per row
    le::DecodeItem pad{};
    pad.token = -1;
    pad.part = -1;
    dec.resize(cap_items, pad);
  }

  // ---- layout: every array 256-byte aligned in one buffer ----
  le_step_plan P{};
  P.cfg = cfg;
  P.n_tokens = static_cast<int32_t>(n_tok);
  P.n_seqs = n_seqs;
  P.n_table = static_cast<int32_t>(n_table);
  P.n_logits = n_logits;
  P.n_decode_items = static_cast<int32_t>(dec.size());
  P.n_chunk_items = static_cast<int32_t>(chk.size());
  P.n_combine_items = 0;  // chunk rows merge inside their launch
  P.n_parts = parts;
  P.max_pos = max_pos;
  P.n_slices = n_slices;
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    const int64_t o = off;
    off = align256(off + std::max<int64_t>(bytes, 4));
    return o;
  };
  P.off_token_ids = take(n_tok * 4);
  P.off_positions = take(n_tok * 4);
  P.off_slots = take(n_tok * 4);
  P.off_token_seq = take(n_tok * 4);
  P.off_tables = take(n_table * 4);
  P.off_table_offset = take(static_cast<int64_t>(n_seqs) * 4);
  P.off_cu_seqlens_q = take(static_cast<int64_t>(n_slices + 1) * 4);
  P.off_seq_lens_k = take(static_cast<int64_t>(n_slices) * 4);
  P.off_logit_rows = take(static_cast<int64_t>(n_logits) * 4);
  P.off_decode_items = take(static_cast<int64_t>(dec.size()) * sizeof(le::DecodeItem));
  P.off_chunk_items = take(static_cast<int64_t>(chk.size()) * sizeof(le::ChunkItem));
  P.off_combine_items = take(0);
  // Each work item's block ids at a fixed stride (decode items, then chunk
  // items), so a workgroup can fetch them in the same memory round trip as
  // its item.
  int32_t ids_stride = 0;
  for (const auto& d : dec) ids_stride = std::max(ids_stride, d.blk_end - d.blk_begin);
  for (const auto& c : chk) ids_stride = std::max(ids_stride, c.blk_end - c.blk_begin);
  if (fixed) ids_stride = std::max(dec_pb, (cfg.table_capacity + parts_cap - 1) / parts_cap);
  ids_stride = (ids_stride + 3) / 4 * 4;
  P.decode_ids_stride = ids_stride;
  P.xcd_local = xcd_local ? 1 : 0;
  P.off_decode_ids = take(static_cast<int64_t>(dec.size() + chk.size()) * ids_stride * 4);
  P.bytes = off;
  P.dev = nullptr;
  if (!host_buf || host_cap < P.bytes) {
    *plan = P;
    return LE_ENOSPACE;
  }

  char* base = static_cast<char*>(host_buf);
  auto arr = [&](int64_t o) { return reinterpret_cast<int32_t*>(base + o); };
  int32_t* token_ids = arr(P.off_token_ids);
  int32_t* positions = arr(P.off_positions);
  int32_t* slots = arr(P.off_slots);
  int32_t* token_seq = arr(P.off_token_seq);
  int32_t* tables = arr(P.off_tables);
  int32_t* table_offset = arr(P.off_table_offset);
  int32_t* cu_q = arr(P.off_cu_seqlens_q);
  int32_t* lens_k = arr(P.off_seq_lens_k);
  int32_t* logit_rows = arr(P.off_logit_rows);

  int32_t nt = 0;
  for (int s = 0; s < n_seqs; s++) {
    const le_step_slice& f = slices[seq_first_slice[s]];
    table_offset[s] = nt;
    if (f.num_blocks) std::memcpy(tables + nt, f.blocks, sizeof(int32_t) * f.num_blocks);
    const int32_t width = fixed ? cfg.table_capacity : f.num_blocks;
    for (int32_t j = f.num_blocks; j < width; j++) tables[nt + j] = -1;
    nt += width;
  }
  int32_t t = 0, r = 0;
  cu_q[0] = 0;
  for (int i = 0; i < n_slices; i++) {
    const le_step_slice& s = slices[i];
    // Slots come from the table of the sequence (its first slice), as the
    // reference reads them from the Sequence object.
    const le_step_slice& f = slices[seq_first_slice[slice_seq[i]]];
    for (int k = 0; k < s.len; k++) {
      const int pos = s.start + k;
      token_ids[t] = s.tokens[pos];
      positions[t] = pos;
      token_seq[t] = slice_seq[i];
      slots[t] = static_cast<int32_t>(static_cast<int64_t>(f.blocks[pos / bs]) * bs + pos % bs);
      t++;
    }
    if (s.needs_logits) logit_rows[r++] = t - 1;
    cu_q[i + 1] = t;
    lens_k[i] = s.start + s.len;
  }
  if (!dec.empty()) {
    std::memcpy(base + P.off_decode_items, dec.data(), dec.size() * sizeof(le::DecodeItem));
    int32_t* ids = arr(P.off_decode_ids);
    for (size_t k = 0; k < dec.size(); k++) {
      const le::DecodeItem& d = dec[k];
      int32_t* row = ids + k * static_cast<size_t>(ids_stride);
      for (int j = 0; j < ids_stride; j++)
        row[j] = j < d.blk_end - d.blk_begin ? tables[d.table_off + d.blk_begin + j] : -1;
    }
  }
  if (!chk.empty()) {
    std::memcpy(base + P.off_chunk_items, chk.data(), chk.size() * sizeof(le::ChunkItem));
    int32_t* ids = arr(P.off_decode_ids) + dec.size() * static_cast<size_t>(ids_stride);
    for (size_t k = 0; k < chk.size(); k++) {
      const le::ChunkItem& c = chk[k];
      const int32_t toff = table_offset[c.seq];
      int32_t* row = ids + k * static_cast<size_t>(ids_stride);
      for (int j = 0; j < ids_stride; j++)
        row[j] = j < c.blk_end - c.blk_begin ? tables[toff + c.blk_begin + j] : -1;
    }
  }
  *plan = P;
  return LE_OK;
}

int le_plan_upload(le_step_plan* plan, const void* host_buf, void* dev_buf, hipStream_t stream) {
  if (!plan || !host_buf || !dev_buf || plan->bytes <= 0) return LE_EINVAL;
  const hipError_t e = hipMemcpyAsync(dev_buf, host_buf, static_cast<size_t>(plan->bytes),
                                      hipMemcpyHostToDevice, stream);
  if (e != hipSuccess) return static_cast<int>(e);
  plan->dev = dev_buf;
  return LE_OK;
}

}  // extern "C"
