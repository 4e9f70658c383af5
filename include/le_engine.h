/*
 * llm-engine on MI355X: host engine around the hot path (C ABI).
 *
 * The reference's callers of the path, kept here so that end-to-end runs go
 * through the same kernels: the block allocator + scheduler
 * (include/engine/kv_cache.h, include/engine/scheduler.h), and a device model
 * whose forward (reference: CudaModel::forward, src/model/cuda/cuda_model.cu:
 * 324-429) packs each step with le_plan_step, scatters K/V with
 * le_kv_cache_write and attends with le_ragged_paged_attention. GEMMs are
 * rocBLAS calls; greedy selection runs on the device.
 *
 * Status convention as in llm_engine_amd.h. Handles are opaque; nothing here
 * is thread-safe (the reference's engine thread is the only caller).
 */
#ifndef LE_ENGINE_H
#define LE_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#include "llm_engine_amd.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scheduler (reference: Scheduler / SchedulerConfig, scheduler.h:22-95) ---- */
typedef struct le_sched_config {
  int32_t continuous;             /* 1 = continuous batching, 0 = static baseline */
  int32_t max_num_seqs;
  int32_t max_num_batched_tokens;
  int32_t prefill_chunk_size;
  int32_t admission_lookahead;
  int32_t starvation_wait_steps;
  int32_t watermark_blocks;       /* -1 = one block per resident sequence */
  int32_t reserved_;
  double max_queue_wait_seconds;  /* 0 = no deadline */
} le_sched_config;

/* The scheduler and block allocator driven by a deterministic fake model
 * (token = 1000 + step counter), recorded step by step. Same arguments and
 * output stream as the reference's trace harness (oracle/ref_harness.cpp), so
 * the two can be compared directly:
 *   per step: n_slices, then per slice: seq_id, start, len, needs_logits,
 *   is_prefill, num_blocks, blocks[...]; then -1; then per sequence: n, tokens.
 * Returns the number of int32 written, or -(needed) if out_cap is too small. */
int64_t le_sched_trace(int num_blocks, int block_size, int prefix_caching,
                       const le_sched_config* cfg, int fragment_blocks, int n_seqs,
                       const int32_t* prompt_lens, const int32_t* prompts_flat,
                       const int32_t* max_tokens, int max_steps, int32_t* out, int64_t out_cap);

/* A steppable scheduler for callers that run their own model (the CPU oracle,
 * a Python loop): Scheduler::schedule / on_step_done (scheduler.h:58-95).
 * Slices returned by le_sched_step point into the scheduler's sequences and
 * stay valid until the next le_sched_done. Sequence ids are the caller's. */
typedef struct le_sched le_sched;
le_sched* le_sched_create(int num_blocks, int block_size, int prefix_caching,
                          const le_sched_config* cfg, int fragment_blocks);
void le_sched_destroy(le_sched* s);
int le_sched_add(le_sched* s, int64_t id, const int32_t* prompt, int n, int max_tokens);
int le_sched_has_work(const le_sched* s);
/* n_slices = 0 when nothing is runnable. LE_ENOSPACE if cap is too small. */
int le_sched_step(le_sched* s, le_step_slice* out, int cap, int* n_slices);
/* sampled[i]: token of the i-th slice with needs_logits of the last step. */
int le_sched_done(le_sched* s, const int32_t* sampled, int n);
/* Generated tokens of sequence `id` (count returned; at most cap written). */
int le_sched_generated(const le_sched* s, int64_t id, int32_t* out, int cap);

/* ---- device model (reference: Model / make_cuda_model, model.h:16-85) ---- */
typedef struct le_model_desc {
  int32_t hidden, inter, layers, q_heads, kv_heads, head_dim, vocab, max_pos;
  float eps, theta;
  int32_t tie_word_embeddings;
  int32_t dtype;       /* le_dtype of weights and activations on the device */
  int32_t kv_dtype;    /* le_dtype of the paged K/V cache */
  int32_t attention;   /* LE_ATTN_RAGGED (0): le_ragged_paged_attention_qkv over the packed
                          step; LE_ATTN_REFERENCE (1): le_rope_kv_cache_write, then the
                          reference-shaped le_attention_decode on the packed arrays */
  /* host fp32 weights, row-major, nn.Linear layout [out][in] */
  const float* embed;       /* [vocab][hidden] */
  const float* final_norm;  /* [hidden] */
  const float* lm_head;     /* [vocab][hidden]; ignored when tied */
  const float* const* in_norm;   /* per layer [hidden] */
  const float* const* post_norm; /* per layer [hidden] */
  const float* const* wq;        /* [q_heads*head_dim][hidden] */
  const float* const* wk;        /* [kv_heads*head_dim][hidden] */
  const float* const* wv;
  const float* const* wo;        /* [hidden][q_heads*head_dim] */
  const float* const* bq;        /* per layer, or NULL (no qkv bias) */
  const float* const* bk;
  const float* const* bv;
  const float* const* wgate;     /* [inter][hidden] */
  const float* const* wup;
  const float* const* wdown;     /* [hidden][inter] */
  /* bf16 models fold both RMSNorms of a layer into the GEMMs around them
   * (norm weights in the weight columns, residual adds in the O and down
   * projections' epilogues, row scales in the SiLU kernel and the attention
   * launch). Nonzero: keep the norm launches (the fp32 model's order of
   * operations), e.g. to compare the two. */
  int32_t unfused_norms;
} le_model_desc;

#define LE_ATTN_RAGGED 0
#define LE_ATTN_REFERENCE 1

typedef struct le_model le_model;

/* Uploads the weights, builds RoPE tables, allocates one K/V cache pair per
 * layer of num_blocks * block_size slots. NULL on failure (*status set). */
le_model* le_model_create(const le_model_desc* desc, int num_blocks, int block_size, int* status);
void le_model_destroy(le_model* m);

/* Decode steps (one row per sequence, every row sampled, no logits copied
 * back) replayed from HIP graphs: per row count, the first step runs eagerly,
 * the second is captured (plan upload, every layer's GEMMs and kernels, the
 * greedy selection and the token copy), later ones replay it with the new
 * plan packed in a fixed layout (le_plan_config.table_capacity). Results are
 * those of the eager path. Off by default. le_model_graph_replays counts the
 * replays so far. */
int le_model_set_decode_graph(le_model* m, int enable);
int64_t le_model_graph_replays(const le_model* m);
/* Decode steps that ran eagerly although graph replay was on: the step's
 * fixed-layout plan was rejected (a table longer than max_pos allows) or
 * the capture failed (after which every step runs eagerly). */
int64_t le_model_eager_fallbacks(const le_model* m);

/* le_model_set_plan_flags sets le_plan_config.flags of the model's plans
 * (default LE_PLAN_XCD_LOCAL: the model launches on its own stream, without a
 * CU mask; LE_PLAN_TWO_LAUNCHES: the tests check that launch shape end to
 * end; 0: write-through partials). */
int le_model_set_plan_flags(le_model* m, int32_t flags);


/* One step: slices in scheduler order. tokens_out receives the greedy token
 * of every slice with needs_logits (first maximum wins); logits_out, if not
 * NULL, receives their fp32 logits [n_logits][vocab]. */
int le_model_forward(le_model* m, const le_step_slice* slices, int n_slices, int32_t* tokens_out,
                     float* logits_out);

/* ---- greedy selection on the device (reference: Sampler::argmax,
 *      sampler.cpp:9-13, run on the host over copied-back logits) ----
 * out[r] = index of the first maximum of logits[r][0..vocab) (fp32, rows
 * contiguous), exactly as the reference's loop picks it: start at element 0,
 * move only to a strictly greater value. So ties go to the lowest index, a
 * NaN is never chosen past element 0, and a row whose element 0 is NaN (or
 * with no greater value) gives 0. One launch for all rows. */
int le_argmax_rows(const float* logits, int rows, int vocab, int32_t* out, hipStream_t stream);

/* ---- serving loop (reference: greedy_run, test_cuda_invariance.cpp:90-143,
 *      and Engine::run_loop, engine.cpp:246) ---- */
typedef struct le_run_stats {
  int64_t steps, prompt_tokens, decode_tokens, preemptions;
  double seconds, decode_seconds;  /* wall time of the loop; of steps with no prefill */
  int64_t decode_steps;            /* steps with no prefill */
  int64_t decode_step_tokens;      /* tokens sampled in those steps */
  double ttft_mean_s;              /* arrival (or start) to first token, mean over sequences */
  double latency_mean_s;           /* arrival (or start) to last token, mean over sequences */
  double plan_seconds;             /* host time in le_plan_step + le_plan_upload, all steps */
  int64_t decode_context_tokens;   /* keys attended (pos + 1) summed over the rows of those steps */
} le_run_stats;

/* Pool preparation code (the fragment_blocks argument of le_sched_trace,
 * le_sched_create and le_run_greedy). n >= 0: the reference's fragmentation
 * recipe (test_cuda_invariance.cpp:98-105) - allocate n one-block sequences,
 * free every other one. LE_POOL_SHUFFLED | seed (seed < 2^30): the free list
 * in a seeded random order, so every table is drawn from a random permutation
 * of the pool (not in the reference; BASELINE config 1's fragmented tables). */
#define LE_POOL_SHUFFLED (1 << 30)

/* Greedy generation of n_seqs prompts through the scheduler and the model.
 * arrival_s (NULL = all at t=0) delays each request until that many seconds
 * after the start (Poisson arrivals for serving runs). fragment_blocks
 * prepares the pool (LE_POOL_SHUFFLED above). gen_out receives, per sequence, max_tokens[i] ids (unused
 * entries -1). */
int le_run_greedy(le_model* m, const le_sched_config* cfg, int prefix_caching, int fragment_blocks,
                  int n_seqs, const int32_t* prompt_lens, const int32_t* prompts_flat,
                  const int32_t* max_tokens, const double* arrival_s, int32_t* gen_out,
                  le_run_stats* stats);

#ifdef __cplusplus
}
#endif
#endif /* LE_ENGINE_H */
