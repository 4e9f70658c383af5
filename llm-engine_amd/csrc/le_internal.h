// Internal launch functions behind the C ABI in include/llm_engine_amd.h.
// Argument validation happens in abi.cpp; these assume valid shapes.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace le {

// Split-K partial result of one (row, q head, context partition): the
// unnormalised accumulator, and the running max (log2 domain) and sum.
struct PartialLayout {
  float* acc;         // [n_parts][q_heads][head_dim]
  float2* ml;         // [n_parts][q_heads]  (m, l)
  unsigned long long* counters;  // [n_rows][kv_heads] arrivals; zero between launches
};

// Decode work item: query row `token` (position `pos`, block table starting
// at tables + table_off) over blocks [blk_begin, blk_end) of its table. The
// row's position and table offset travel in the item so a workgroup reaches
// its first K/V load after one dependent read. part < 0: the row has a single
// partition and the kernel writes the normalised output itself. Otherwise the
// item writes partial `part`, and the last of the row's n_parts items to
// arrive (per kv head) merges partials [part_begin, part_begin + n_parts).
struct DecodeItem {
  int32_t token, pos, table_off, blk_begin, blk_end, part, part_begin, n_parts;
};

// Chunk work item: query rows [tok_begin, tok_begin + n_q) (consecutive
// positions of one sequence, at most 32) over key blocks [blk_begin, blk_end)
// of its table, partition `part` of the tile's part_stride partitions. Row
// tok_begin + i writes partial part0 + i * part_stride, or, when part0 < 0,
// its normalised output directly; the last partition of the tile to arrive
// (per kv head) merges partials [part0 - part + i * part_stride, ... +
// part_stride) of each row.
struct ChunkItem {
  int32_t tok_begin, n_q, blk_begin, blk_end, part0, part_stride, seq, part;
  // keys of [blk_begin * block_size, ...) that hold a live position (at most
  // the tile's last position + 1): rows past it are never read
  int32_t key_live;
};

// Element types are passed as le_dtype codes: 0 fp32, 1 bf16, 2 fp16.
constexpr int kDtF32 = 0, kDtBF16 = 1, kDtF16 = 2;

hipError_t kv_cache_write(const void* k, const void* v, int src_dtype, const int32_t* slots,
                          void* kc, void* vc, int cache_dtype, int n_tokens, int kv_dim,
                          int64_t num_slots, hipStream_t stream);
hipError_t rope_kv_cache_write(const void* qkv, int act_dtype, int64_t row_stride, const float* bias,
                               const int32_t* positions, const int32_t* slots, const float* cos_t,
                               const float* sin_t, int max_pos, int n_tokens, int q_heads,
                               int kv_heads, int head_dim, void* q_out, void* kc, void* vc,
                               int cache_dtype, int64_t num_slots, hipStream_t stream,
                               const void* rms_x = nullptr, int rms_hidden = 0, float rms_eps = 0.f);

struct DecodeParams {
  const void* q;
  const void* k_cache;
  const void* v_cache;
  const int32_t* tables;
  const int32_t* table_offset;
  const int32_t* token_seq;
  const int32_t* token_pos;
  void* out;
  PartialLayout parts;
  // With a plan and a pure decode step: the step's new K/V rows ([n_tokens]
  // [kv_heads * head_dim], element type new_dtype). The last partition
  // of each row stores its row (for its kv head) at slots[token] before any
  // K/V load of the launch reads it. Null: the rows are already in the cache.
  const void* k_new;
  const void* v_new;
  const int32_t* slots;
  int new_dtype;
  int64_t num_slots;
  // Rows straight from the stacked QKV projection (rope_max_pos > 0): q and
  // the new K/V rows are read at rope_row_stride elements per token (q, k_new
  // and v_new point at row 0's q, k and v parts, all in the activation type);
  // the bias (fp32 [q | k | v], may be null) is added and rounded to the
  // activation type, then q and k rotate by the row's position (tables
  // [rope_max_pos][head_dim / 2]) exactly as rope_kv_cache_write computes
  // them. A row whose position is outside the tables attends with q = 0 and
  // stores nothing (as rope_kv_cache_write writes zeros and skips the store).
  int64_t rope_row_stride;
  const float* rope_bias;
  const float* rope_cos;
  const float* rope_sin;
  int rope_max_pos;
  // With rope rows: the pre-attention RMSNorm folded into the QKV projection.
  // rms_x (act dtype, [tokens][rms_hidden]) is the residual stream the rows
  // were projected from; each row is scaled by 1/sqrt(mean(x^2) + rms_eps)
  // before its bias. Null: the rows are already normalised.
  const void* rms_x;
  int rms_hidden;
  float rms_eps;
  const DecodeItem* items;  // null: one item per (token, split) with `nsplit` splits
  const int32_t* item_ids;  // with items: block ids of item i at item_ids[i * ids_stride + j]
  int ids_stride;
  int n_rows;               // items, or tokens when items is null
  int nsplit;
  int q_heads, kv_heads, head_dim, block_size;
  float scale_log2;         // softmax scale * log2(e)
  int64_t num_cache_blocks;
  // With items: every partition of a split row runs on one XCD (the plan's
  // placement, and the dealing confirmed on this device by
  // xcd_placement_holds), so partials go through that XCD's L2 with plain
  // stores.
  int l2_local;
  // Two even rounds of one workgroup per CU or more (a plan of at least 512
  // workgroups with no empty fixed-layout slots): the decode kernel
  // instantiation with no register bound. Otherwise two workgroups per CU.
  int wide;
};

// True when this device deals a launch's workgroups to its XCDs round robin
// (workgroups whose linear ids are equal modulo 8 share an XCD): checked
// once per device with a probe launch, then cached. False while the stream
// is being captured and the device is not checked yet, or on any error.
bool xcd_placement_holds(hipStream_t stream);

hipError_t attention_decode(const DecodeParams& p, int act_dtype, int kv_dtype, hipStream_t stream);

struct ChunkParams {
  const void* q;
  const void* k_cache;
  const void* v_cache;
  const int32_t* tables;
  const int32_t* table_offset;
  const int32_t* token_pos;
  void* out;
  PartialLayout parts;
  const ChunkItem* items;
  const int32_t* item_ids;  // block ids of item i at item_ids[i * ids_stride + j]
  int ids_stride;
  int n_items;
  int q_heads, kv_heads, head_dim, block_size;
  float scale_log2;
  int64_t num_cache_blocks;
  int l2_local;  // split tiles' partitions share an XCD: partials through its L2 (as DecodeParams)
};

hipError_t attention_chunk(const ChunkParams& p, int act_dtype, int kv_dtype, hipStream_t stream);

// A mixed step's chunk rows and decode rows (plan items) in one
// launch: chunk workgroups first, then decode workgroups.
hipError_t attention_ragged(const DecodeParams& d, const ChunkParams& c, int act_dtype, int kv_dtype,
                            hipStream_t stream);

// Split count for the reference-shaped entry point, where the host does not
// know the context lengths: enough workgroups to cover the chip several times.
int decode_nsplit(int n_tokens, int kv_heads);

}  // namespace le
