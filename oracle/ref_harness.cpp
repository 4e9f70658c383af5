// C entry points over the reference engine's own CPU sources: TEST
// INFRASTRUCTURE ONLY.
//
// oracle/Makefile compiles this file together with the reference's
// src/kv_cache/block_allocator.cpp, src/scheduler/scheduler.cpp and
// src/model/sampler.cpp, straight from /root/reference, into
// oracle/_ref/libref.so. The header-only parts (include/engine/ops.h,
// tensor.h, kv_cache.h) are used in place. The result is used only to check
// the C restatement in oracle/oracle.c and to write the fixtures under
// tests/golden/. Nothing here is copied from the reference: this file only
// calls it.
//
// The reference's forward pass (src/model/cpu/cpu_model.cpp) is not built:
// it needs the safetensors/config readers, which need nlohmann/json, an
// external library. Its per-op pieces all live in ops.h and are built here.
#include <cstdint>
#include <cstring>
#include <memory>
#include <vector>

#include "engine/kv_cache.h"
#include "engine/ops.h"
#include "engine/sampler.h"
#include "engine/scheduler.h"
#include "engine/tensor.h"

using namespace engine;

extern "C" {

uint16_t ref_f32_to_bf16(float f) { return f32_to_bf16(f); }
float ref_bf16_to_f32(uint16_t h) { return bf16_to_f32(h); }
uint16_t ref_f32_to_f16(float f) { return f32_to_f16(f); }
float ref_f16_to_f32(uint16_t h) { return f16_to_f32(h); }

int64_t ref_slot(const int32_t* blocks, int num_blocks, int pos, int block_size) {
  BlockTable bt;
  bt.blocks.assign(blocks, blocks + num_blocks);
  return bt.slot(pos, block_size);
}

void ref_rmsnorm(const float* x, const float* w, float* out, int rows, int cols, float eps) {
  ref::rmsnorm(x, w, out, rows, cols, eps);
}

void ref_rope_tables(int head_dim, int max_positions, float theta, float* cos_t, float* sin_t) {
  ref::RopeTables t;
  t.build(head_dim, max_positions, theta);
  std::memcpy(cos_t, t.cos.data(), t.cos.size() * sizeof(float));
  std::memcpy(sin_t, t.sin.data(), t.sin.size() * sizeof(float));
}

void ref_rope_inplace(float* x, int heads, int head_dim, int pos, int max_positions, float theta) {
  ref::RopeTables t;
  t.build(head_dim, max_positions, theta);
  ref::rope_inplace(x, heads, head_dim, pos, t);
}

void ref_silu_mul(float* gate, const float* up, size_t n) { ref::silu_mul(gate, up, n); }

int32_t ref_argmax(const float* logits, int vocab) { return Sampler::argmax(logits, vocab); }

// The (token, head) loop of cpu_model.cpp:173-185 around ref::paged_attention_head,
// over the concatenated-table layout (tables + table_offset + token_seq).
// table_len[s] is the number of blocks of distinct sequence s.
void ref_paged_attention(const float* q, int q_stride, const float* k_cache, const float* v_cache,
                         const int32_t* tables, const int32_t* table_offset,
                         const int32_t* table_len, const int32_t* token_seq,
                         const int32_t* token_pos, int n_tokens, int q_heads, int kv_heads,
                         int head_dim, int block_size, float scale, float* out, int out_stride) {
  const int group = q_heads / kv_heads;
  std::vector<float> scratch;
  for (int i = 0; i < n_tokens; i++) {
    const int s = token_seq[i];
    BlockTable bt;
    bt.blocks.assign(tables + table_offset[s], tables + table_offset[s] + table_len[s]);
    for (int h = 0; h < q_heads; h++)
      ref::paged_attention_head(q + static_cast<size_t>(i) * q_stride + h * head_dim, k_cache,
                                v_cache, bt, block_size, token_pos[i], h / group, kv_heads,
                                head_dim, scale,
                                out + static_cast<size_t>(i) * out_stride + h * head_dim, scratch);
  }
}

// Drives the reference Scheduler + KVCacheManager with a deterministic fake
// model (token = 1000 + running counter, as the reference's scheduler tests do)
// and records every step.
//
// Output stream (int32), per step:
//   n_slices, then per slice: seq_id, start, len, needs_logits, is_prefill,
//   num_blocks, blocks[num_blocks]
// followed by a terminator -1, then per sequence: n_tokens, tokens[n_tokens].
// Returns the number of int32 written, or -(needed) if out_cap is too small.
// _ex: also the static-batching switch (continuous = 0), the admission
// lookahead and the starvation bound (scheduler.h:24-37).
int64_t ref_schedule_trace_ex(int num_blocks, int block_size, int prefix_caching,
                              int max_num_seqs, int max_num_batched_tokens, int prefill_chunk_size,
                              int watermark_blocks, int fragment_blocks, int continuous,
                              int admission_lookahead, int starvation_wait_steps, int n_seqs,
                              const int32_t* prompt_lens, const int32_t* prompts_flat,
                              const int32_t* max_tokens, int max_steps, int32_t* out,
                              int64_t out_cap) {
  KVCacheManager kv(num_blocks, block_size, prefix_caching != 0);
  std::vector<BlockTable> held;
  for (int i = 0; i < fragment_blocks; i++) {
    BlockTable bt;
    std::vector<int32_t> one(static_cast<size_t>(block_size) / 2 > 0 ? block_size / 2 : 1,
                             7000 + i);
    if (!kv.allocate_prompt(bt, one).has_value()) break;
    held.push_back(bt);
  }
  for (size_t i = 0; i < held.size(); i += 2) kv.free(held[i]);

  SchedulerConfig cfg;
  cfg.max_num_seqs = max_num_seqs;
  cfg.max_num_batched_tokens = max_num_batched_tokens;
  cfg.prefill_chunk_size = prefill_chunk_size;
  cfg.watermark_blocks = watermark_blocks;
  cfg.continuous = continuous != 0;
  cfg.admission_lookahead = admission_lookahead;
  cfg.starvation_wait_steps = starvation_wait_steps;
  Scheduler sch(cfg, kv);
  std::vector<SequencePtr> seqs;
  size_t off = 0;
  for (int i = 0; i < n_seqs; i++) {
    auto s = std::make_shared<Sequence>();
    s->id = static_cast<uint64_t>(i);
    s->tokens.assign(prompts_flat + off, prompts_flat + off + prompt_lens[i]);
    off += static_cast<size_t>(prompt_lens[i]);
    s->prompt_len = prompt_lens[i];
    s->params.max_tokens = max_tokens[i];
    s->params.temperature = 0.f;
    s->params.ignore_eos = true;
    sch.add(s);
    seqs.push_back(s);
  }

  std::vector<int32_t> rec;
  int32_t next = 1000;
  for (int step = 0; step < max_steps && sch.has_work(); step++) {
    StepInput st = sch.schedule();
    if (st.empty()) break;
    rec.push_back(static_cast<int32_t>(st.slices.size()));
    std::vector<int32_t> sampled;
    for (const auto& sl : st.slices) {
      rec.push_back(static_cast<int32_t>(sl.seq->id));
      rec.push_back(sl.start);
      rec.push_back(sl.len);
      rec.push_back(sl.needs_logits ? 1 : 0);
      rec.push_back(sl.is_prefill ? 1 : 0);
      rec.push_back(sl.seq->block_table.num_blocks());
      for (BlockId b : sl.seq->block_table.blocks) rec.push_back(b);
      if (sl.needs_logits) sampled.push_back(next++);
    }
    sch.on_step_done(st, sampled);
  }
  rec.push_back(-1);
  for (auto& s : seqs) {
    rec.push_back(s->num_tokens());
    for (int32_t t : s->tokens) rec.push_back(t);
  }
  for (size_t i = 1; i < held.size(); i += 2) kv.free(held[i]);
  if (static_cast<int64_t>(rec.size()) > out_cap) return -static_cast<int64_t>(rec.size());
  std::memcpy(out, rec.data(), rec.size() * sizeof(int32_t));
  return static_cast<int64_t>(rec.size());
}

int64_t ref_schedule_trace(int num_blocks, int block_size, int prefix_caching,
                           int max_num_seqs, int max_num_batched_tokens, int prefill_chunk_size,
                           int watermark_blocks, int fragment_blocks, int n_seqs,
                           const int32_t* prompt_lens, const int32_t* prompts_flat,
                           const int32_t* max_tokens, int max_steps, int32_t* out,
                           int64_t out_cap) {
  const SchedulerConfig defaults;
  return ref_schedule_trace_ex(num_blocks, block_size, prefix_caching, max_num_seqs,
                               max_num_batched_tokens, prefill_chunk_size, watermark_blocks,
                               fragment_blocks, defaults.continuous ? 1 : 0,
                               defaults.admission_lookahead, defaults.starvation_wait_steps, n_seqs,
                               prompt_lens, prompts_flat, max_tokens, max_steps, out, out_cap);
}

}  // extern "C"
