/*
 * CPU oracle for the ragged paged-attention path: TEST INFRASTRUCTURE ONLY.
 *
 * A clean-room restatement, in plain C, of the reference engine's fp32 CPU
 * backend for the hot path (llm-engine: include/engine/ops.h,
 * src/model/cpu/cpu_model.cpp, src/model/cuda/cuda_model.cu host packing,
 * include/engine/kv_cache.h, include/engine/tensor.h, src/model/sampler.cpp).
 * Loop and summation orders follow the reference exactly so that results are
 * bit-identical to it (checked against the reference's own sources compiled
 * by oracle/Makefile into oracle/_ref/, and against closed forms).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker or the timed CPU baseline. The
 * product path (llm-engine_amd/) never links, loads or calls it.
 */
#ifndef LE_ORACLE_H
#define LE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar formats: include/engine/tensor.h:20-28 ---- */
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
void orc_f32_to_bf16_n(const float* in, uint16_t* out, size_t n);
void orc_bf16_to_f32_n(const uint16_t* in, float* out, size_t n);
/* ---- scalar formats: include/engine/tensor.h:29-56 (fp16, the reference's __half) ---- */
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
void orc_f32_to_f16_n(const float* in, uint16_t* out, size_t n);
void orc_f16_to_f32_n(const uint16_t* in, float* out, size_t n);

/* ---- paging: include/engine/kv_cache.h:29-31 ---- */
int64_t orc_slot(const int32_t* blocks, int pos, int block_size);

/* ---- step packing: src/model/cuda/cuda_model.cu:434-491 ---- */
typedef struct {
  int64_t seq_key;          /* identity of the owning sequence (the reference dedups by Sequence*) */
  int32_t start, len;       /* tokens [start, start+len) of the sequence */
  int32_t needs_logits;
  int32_t num_blocks;
  const int32_t* blocks;    /* the sequence's block table */
  const int32_t* tokens;    /* the sequence's full token list */
} orc_slice;

/* counts_out = {N tokens, S distinct sequences, T table entries, R logit rows}.
 * Output arrays must hold N (token arrays), S (table_offset), T (tables), R
 * (logit_rows) entries; pass NULL for all outputs to size only. */
void orc_pack_step(const orc_slice* slices, int n_slices, int block_size,
                   int32_t* token_ids, int32_t* positions, int32_t* slots, int32_t* token_seq,
                   int32_t* tables, int32_t* table_offset, int32_t* logit_rows,
                   int32_t counts_out[4]);

/* ---- cache write: src/kernels/store_kv.cu:20-36, cpu_model.cpp:153-157 ---- */
void orc_store_kv(const float* k, const float* v, const int32_t* slots, float* k_cache,
                  float* v_cache, int n_tokens, int kv_dim);
void orc_store_kv_bf16(const float* k, const float* v, const int32_t* slots, uint16_t* k_cache,
                       uint16_t* v_cache, int n_tokens, int kv_dim);

/* ---- attention: include/engine/ops.h:87-111 ---- */
void orc_paged_attention_head(const float* q, const float* k_cache, const float* v_cache,
                              const int32_t* blocks, int block_size, int pos, int kv_head,
                              int kv_heads, int head_dim, float scale, float* out,
                              float* scratch /* >= pos+1 floats */);

/* (token, head) loop of cpu_model.cpp:160-185 over the packed layout of
 * cuda_model.cu:453-491 (tables + table_offset + token_seq + token_pos).
 * q row t, head h at q[t*q_stride + h*head_dim]; same for out. threads<=1 runs
 * serially; the result does not depend on the thread count. */
void orc_paged_attention(const float* q, int q_stride, const float* k_cache, const float* v_cache,
                         const int32_t* tables, const int32_t* table_offset,
                         const int32_t* token_seq, const int32_t* token_pos, int n_tokens,
                         int q_heads, int kv_heads, int head_dim, int block_size, float scale,
                         float* out, int out_stride, int threads);

/* Same, with bf16 caches widened to fp32 on read. */
void orc_paged_attention_bf16kv(const float* q, int q_stride, const uint16_t* k_cache,
                                const uint16_t* v_cache, const int32_t* tables,
                                const int32_t* table_offset, const int32_t* token_seq,
                                const int32_t* token_pos, int n_tokens, int q_heads, int kv_heads,
                                int head_dim, int block_size, float scale, float* out,
                                int out_stride, int threads);

/* ---- layer ops: include/engine/ops.h:22-74, cpu_model.cpp:27-39 ---- */
void orc_rmsnorm(const float* x, const float* weight, float* out, int rows, int cols, float eps);
void orc_rope_tables(int head_dim, int max_positions, float theta, float* cos_t, float* sin_t);
void orc_rope_inplace(float* x, int heads, int head_dim, int pos, const float* cos_t,
                      const float* sin_t);
void orc_silu_mul(float* gate, const float* up, size_t n);
void orc_linear(const float* A, int m, int k, const float* B, int n, const float* bias, float* C,
                int threads);

/* ---- greedy: src/model/sampler.cpp:9-13 ---- */
int32_t orc_argmax(const float* logits, int vocab);

/* ---- whole forward: src/model/cpu/cpu_model.cpp:98-214 ---- */
typedef struct {
  int hidden, inter, layers, q_heads, kv_heads, head_dim, vocab, max_pos;
  float eps, theta;
  int tie_word_embeddings;
  const float* embed;       /* [vocab][hidden] */
  const float* final_norm;  /* [hidden] */
  const float* lm_head;     /* [vocab][hidden], ignored when tied */
  /* per-layer pointer arrays, each `layers` long; bq/bk/bv entries may be NULL */
  const float* const* in_norm;
  const float* const* post_norm;
  const float* const* wq;
  const float* const* wk;
  const float* const* wv;
  const float* const* wo;
  const float* const* bq;
  const float* const* bk;
  const float* const* bv;
  const float* const* wgate;
  const float* const* wup;
  const float* const* wdown;
} orc_model;

/* One step. Caches are per layer, [slots][kv_heads][head_dim]; with kv_bf16
 * they are uint16 bf16 arrays (the fp32 reference with a bf16 KV store),
 * otherwise float. rope_cos/sin are orc_rope_tables(head_dim, max_pos, theta).
 * logits: [R][vocab]. */
void orc_forward(const orc_model* m, const float* rope_cos, const float* rope_sin,
                 void* const* k_caches, void* const* v_caches, int kv_bf16,
                 const int32_t* token_ids, const int32_t* positions, const int32_t* slots,
                 const int32_t* token_seq, const int32_t* tables, const int32_t* table_offset,
                 int n_tokens, const int32_t* logit_rows, int n_logits, int block_size,
                 float* logits, int threads);

/* orc_forward that also records the residual stream: resid, when not NULL,
 * receives [layers+1][n_tokens][hidden] floats (after the embedding, then
 * after each layer), the capture of test_cpu_model.cpp:112-125. */
void orc_forward_trace(const orc_model* m, const float* rope_cos, const float* rope_sin,
                       void* const* k_caches, void* const* v_caches, int kv_bf16,
                       const int32_t* token_ids, const int32_t* positions, const int32_t* slots,
                       const int32_t* token_seq, const int32_t* tables,
                       const int32_t* table_offset, int n_tokens, const int32_t* logit_rows,
                       int n_logits, int block_size, float* logits, int threads, float* resid);

#ifdef __cplusplus
}
#endif
#endif
