/*
 * llm-engine on MI355X: C ABI of the ragged continuous-batching hot path.
 *
 * This header replaces the CUDA launcher boundary of the reference engine,
 * include/engine/cuda_kernels.h:17-64 (namespace engine, guarded by
 * ENGINE_CUDA). Every entry point here is plain C: raw device pointers, sizes,
 * a dtype tag and a hipStream_t. Nothing allocates device memory; scratch comes
 * in through an explicit workspace argument whose size a *_workspace_size call
 * reports. Exceptions never cross this boundary.
 *
 * Attention workspaces: zero-fill a workspace once, before its first use;
 * every launch leaves it that way again. Its first 512 KiB hold arrival
 * counters (64-bit, one per (row, kv head); at most 65536 of them, else
 * LE_EUNSUPPORTED) at the same place for every plan, then the split-K
 * partials, so one workspace of the largest size needed can serve steps of
 * any shape. Launches that share a workspace must be ordered on one stream.
 *
 * Return value of every int-returning call:
 *     0            LE_OK
 *     < 0          a LE_E* code: bad shape or argument, nothing was launched
 *     > 0          a hipError_t from the launch (hipGetLastError)
 * The reference launchers return void and throw std::runtime_error on bad
 * shapes (attention_decode_gqa.cu:211-224); the C++ engine in this repository
 * turns a non-zero status back into that exception.
 *
 * Layouts (identical to the reference, cuda_model.cu:276-285 and
 * kv_cache.h:21-32):
 *   K and V cache, per layer:  [num_blocks * block_size][kv_heads][head_dim]
 *   slot(pos)               =  block_table[pos / block_size] * block_size
 *                              + pos % block_size
 *   q, out                  :  [n_tokens][q_heads][head_dim], row-contiguous
 *   new k, v rows           :  [n_tokens][kv_heads * head_dim]
 * Element types: LE_F32 (float), LE_BF16 (raw bf16 bits, uint16) or LE_F16
 * (raw IEEE binary16 bits, uint16; the reference's __half).
 */
#ifndef LLM_ENGINE_AMD_H
#define LLM_ENGINE_AMD_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LE_OK 0
#define LE_EINVAL (-1)       /* a pointer, size or shape is invalid */
#define LE_EUNSUPPORTED (-2) /* valid, but outside what the kernels are built for */
#define LE_ENOSPACE (-3)     /* a caller buffer (host plan buffer, workspace) is too small */
#define LE_ETOOLARGE (-5)    /* the step needs more scratch than le_ragged_paged_attention_noalloc
                                has (le_noalloc_scratch_bytes); nothing was launched */
#define LE_EDEVICE (-4)      /* a device library call (rocBLAS) failed; a failed HIP call
                                returns its positive hipError_t instead */

typedef enum le_dtype { LE_F32 = 0, LE_BF16 = 1, LE_F16 = 2 } le_dtype;

/* Library version and build identification (for logs). */
const char* le_version(void);
/* Human-readable name of a status code. */
const char* le_status_string(int status);

/* ------------------------------------------------------------------------
 * (2) K/V cache-write scatter.
 * Replaces launch_store_kv (cuda_kernels.h:43-45, store_kv.cu:20-36):
 *     k_cache[slot_mapping[t]][j] = k[t][j],  v likewise,  j < kv_dim.
 * src and cache dtypes may differ (fp32 rows into a bf16 cache round to
 * nearest even). A negative slot skips the token (padding). Slots at or
 * beyond num_slots are rejected on the device (the row is not written).
 * kv_dim must be a multiple of 8.
 * ------------------------------------------------------------------------ */
int le_kv_cache_write(const void* k, const void* v, le_dtype src_dtype,
                      const int32_t* slot_mapping, void* k_cache, void* v_cache,
                      le_dtype cache_dtype, int n_tokens, int kv_dim, int64_t num_slots,
                      hipStream_t stream);

/* ------------------------------------------------------------------------
 * (2) The scatter fused with what produces its rows.
 * Replaces the reference's bias + RoPE + cache-write sequence of each layer
 * (cuda_model.cu:358-368: launch_add_bias x3, launch_rope on q and k,
 * launch_store_kv; kernels elementwise.cu:40, rope.cu:53, store_kv.cu:31)
 * with one launch over the fused QKV projection output:
 *     row t of qkv = [ q (q_heads*head_dim) | k (kv_heads*head_dim) | v (kv_heads*head_dim) ]
 *     x += bias (if not NULL, fp32 [q_dim + 2*kv_dim]; rounded to act_dtype as
 *                the separate add would store it)
 *     q, k rotated by RoPE at positions[t] (rotate_half pairing i <-> i+half,
 *        a' = a*cos - b*sin, b' = b*cos + a*sin, no fused multiply-add)
 *     q_out[t] = q  (contiguous [n_tokens][q_heads*head_dim], act_dtype)
 *     k_cache[slots[t]] = k, v_cache[slots[t]] = v  (cache_dtype)
 * cos/sin tables are fp32 [max_positions][head_dim/2]. A negative slot skips
 * the K/V write (padding), as does a slot >= num_slots. A position outside
 * [0, max_positions) zero-fills that token's q row and skips its K/V write.
 * head_dim a multiple of 8; qkv_row_stride (elements) >= (q_heads+2*kv_heads)*head_dim
 * and a multiple of 8; all buffers 16-byte aligned.
 * ------------------------------------------------------------------------ */
int le_rope_kv_cache_write(const void* qkv, le_dtype act_dtype, int64_t qkv_row_stride,
                           const float* bias, const int32_t* positions,
                           const int32_t* slot_mapping, const float* cos_table,
                           const float* sin_table, int max_positions, int n_tokens, int q_heads,
                           int kv_heads, int head_dim, void* q_out, void* k_cache, void* v_cache,
                           le_dtype cache_dtype, int64_t num_slots, hipStream_t stream);

/* ------------------------------------------------------------------------
 * (3)(4) Paged attention, reference-shaped.
 * Replaces launch_attention_decode and launch_attention_decode_gqa
 * (cuda_kernels.h:50-64, attention_decode.cu:45-161,
 * attention_decode_gqa.cu:87-232). Same arguments and the same result:
 * token t attends over positions 0..token_pos[t] of sequence token_seq[t],
 * whose block table starts at block_tables + table_offset[token_seq[t]];
 * kv_head = head / (q_heads / kv_heads). One K/V read serves the whole GQA
 * group. The context of each token is split across workgroups (split-K), the
 * partial results merged inside the launch by the last partition to finish,
 * so `workspace` must hold le_attention_decode_workspace_size(n_tokens,
 * q_heads, kv_heads, head_dim) bytes.
 * q/out dtype `act_dtype`, caches `kv_dtype`. head_dim 64 or 128;
 * q_heads / kv_heads <= 8; block_size a multiple of 8 (16 in every config).
 * num_cache_blocks bounds the block ids read from the tables.
 * ------------------------------------------------------------------------ */
size_t le_attention_decode_workspace_size(int n_tokens, int q_heads, int kv_heads, int head_dim);

int le_attention_decode(const void* q, le_dtype act_dtype, const void* k_cache,
                        const void* v_cache, le_dtype kv_dtype, const int32_t* block_tables,
                        const int32_t* table_offset, const int32_t* token_seq,
                        const int32_t* token_pos, void* out, int n_tokens, int q_heads,
                        int kv_heads, int head_dim, int block_size, float scale,
                        int64_t num_cache_blocks, void* workspace, size_t workspace_bytes,
                        hipStream_t stream);

/* ------------------------------------------------------------------------
 * (1) Ragged step packing.
 * Replaces CudaModel::flatten + upload_step_indices (cuda_model.cu:434-491):
 * the scheduler's slices (prefill chunks first, then decode tokens,
 * scheduler.cpp:164-211) become ONE buffer holding token ids, positions,
 * slot mapping, token->sequence, concatenated block tables + offsets,
 * cu_seqlens_q, seq_lens_k, logit rows and the attention work lists, uploaded
 * with one hipMemcpyAsync per step and shared by every layer.
 * ------------------------------------------------------------------------ */
typedef struct le_step_slice {
  int64_t seq_key;       /* sequence identity; slices with one key share one table */
  int32_t start;         /* first position computed by this slice */
  int32_t len;           /* number of tokens (1 for decode) */
  int32_t needs_logits;  /* last token produces a logits row */
  int32_t num_blocks;    /* entries of `blocks` */
  const int32_t* blocks; /* the sequence's block table */
  const int32_t* tokens; /* the sequence's token ids, at least start+len of them */
} le_step_slice;

typedef struct le_plan_config {
  int32_t q_heads, kv_heads, head_dim, block_size;
  int32_t kv_dtype;            /* le_dtype of the cache the plan will be run against */
  int32_t partition_tokens;    /* split-K partition of decode rows; 0 = default */
  int32_t chunk_q_tile;        /* query rows per chunk tile (16 or 32); 0 = default (32) */
  int32_t chunk_partition_tokens; /* key partition of chunk tiles; 0 = default */
  int32_t flags;               /* LE_PLAN_* bits below; 0 = the defaults */
  int32_t table_capacity;      /* 0: tables packed exactly. > 0: a fixed layout for a step of
                                  decode rows only, so launches captured in a HIP graph can be
                                  replayed for later steps with the same number of rows: every
                                  sequence's table gets table_capacity entries, every row
                                  partition_tokens-sized partitions (partition_tokens must be
                                  given), and the work lists, partials and every array offset
                                  depend only on the row count */
} le_plan_config;

/* le_plan_config.flags. LE_PLAN_TWO_LAUNCHES selects a slower, equivalent
 * launch shape (the tests use it to check that launch shapes agree);
 * LE_PLAN_XCD_LOCAL a faster exchange of partials under a precondition. */
#define LE_PLAN_TWO_LAUNCHES 2  /* a mixed step runs its decode and chunk rows as two
                                   launches instead of one */
#define LE_PLAN_XCD_LOCAL 4     /* opt in to the XCD-local exchange of split rows' partials
                                   (no counterpart in the reference, whose GPU has one L2):
                                   the plan places all partitions of a split decode row or
                                   chunk tile at workgroup ids equal modulo 8, and the launch
                                   stores their partials into one XCD's L2 with plain stores
                                   instead of write-through ones (config 3: 22.9 -> 20.6 us per
                                   launch). Precondition: the device deals a launch's workgroups
                                   to its XCDs round robin, which holds in every compute
                                   partition mode but not on streams with a CU mask; do not use
                                   the flag on such streams. The dealing is probed once per device
                                   (a small launch, outside stream capture); where it does not
                                   hold, or before it is probed inside a capture, the launch
                                   stores write-through as without the flag. Ignored by
                                   fixed-layout plans. */

typedef struct le_step_plan {
  le_plan_config cfg;
  int32_t n_tokens;      /* packed query rows */
  int32_t n_seqs;        /* distinct sequences (tables), first-seen order */
  int32_t n_table;       /* entries of the concatenated block tables */
  int32_t n_logits;      /* logit rows */
  int32_t n_decode_items, n_chunk_items;
  int32_t n_combine_items; /* always 0: split rows merge inside their launch (kept for layout) */
  int32_t n_parts;
  int32_t max_pos;
  int32_t n_slices;      /* entries of cu_seqlens_q minus one, and of seq_lens_k */
  /* byte offsets of each array inside the packed buffer */
  int64_t off_token_ids, off_positions, off_slots, off_token_seq, off_tables,
      off_table_offset, off_cu_seqlens_q, off_seq_lens_k, off_logit_rows, off_decode_items,
      off_chunk_items, off_combine_items;
  int64_t off_decode_ids;     /* block ids of each decode item, then of each chunk item,
                                 decode_ids_stride apart */
  int32_t decode_ids_stride;  /* entries per work item in that array (padded with -1) */
  int32_t xcd_local;          /* 1: every split row's or tile's partitions sit at item indices
                                 equal modulo 8 (LE_PLAN_XCD_LOCAL honoured) */
  int64_t bytes;         /* total size of the packed buffer */
  const void* dev;       /* device copy, set by le_plan_upload */
} le_step_plan;

/* Packs a step into host_buf (pinned memory recommended). If host_cap is too
 * small, returns LE_ENOSPACE with plan->bytes set to the size needed. */
int le_plan_step(const le_step_slice* slices, int n_slices, const le_plan_config* cfg,
                 void* host_buf, int64_t host_cap, le_step_plan* plan);

/* One async copy of the packed buffer to dev_buf (>= plan->bytes), then
 * plan->dev = dev_buf. The host buffer must stay alive until the copy ends. */
int le_plan_upload(le_step_plan* plan, const void* host_buf, void* dev_buf,
                   hipStream_t stream);

/* Device address of one packed array (e.g. plan->off_slots). */
static inline const int32_t* le_plan_dev_array(const le_step_plan* plan, int64_t off) {
  return (const int32_t*)((const char*)plan->dev + off);
}

/* ------------------------------------------------------------------------
 * (3)(4) Ragged paged attention over a packed step.
 * Decode rows (slices of length 1) run the bandwidth kernel: one workgroup per
 * (row, kv head, context partition), each K/V row read once for the whole
 * GQA group. Prefill-chunk rows run the MFMA tile kernel (bf16 / fp16 tiles
 * for 16-bit caches, fp32 tiles for an fp32 cache), with a causal mask by
 * absolute position against the cached prefix. Split rows are merged inside
 * their launch. The result equals le_attention_decode on the same step.
 * ------------------------------------------------------------------------ */
size_t le_ragged_workspace_size(const le_step_plan* plan);

int le_ragged_paged_attention(const void* q, le_dtype act_dtype, const void* k_cache,
                              const void* v_cache, le_dtype kv_dtype, int64_t num_cache_blocks,
                              const le_step_plan* plan, float scale, void* out, void* workspace,
                              size_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------------------------
 * (3)(4) Ragged paged attention that allocates nothing and takes no
 * workspace. No counterpart in the reference: it is for callers that cannot
 * allocate device memory or pass a workspace (code under HIP graph capture,
 * tight serving loops, harnesses that forbid allocation). Same arguments and
 * the same result as le_ragged_paged_attention, bit for bit, without
 * `workspace`: the split-K partials and arrival counters live in a static
 * device array of le_noalloc_scratch_bytes() (32 MiB), one per GPU, held
 * until the process ends. A step whose le_ragged_workspace_size exceeds it
 * returns LE_ETOOLARGE and launches nothing. The first call on a device
 * clears the array's counters with a fill kernel on `stream`; every launch
 * leaves them at zero. All calls on one GPU share its array: calls that
 * overlap on one GPU (different streams, different threads) race; order
 * them on one stream.
 * ------------------------------------------------------------------------ */
size_t le_noalloc_scratch_bytes(void);

int le_ragged_paged_attention_noalloc(const void* q, le_dtype act_dtype, const void* k_cache,
                                      const void* v_cache, le_dtype kv_dtype, int64_t num_cache_blocks,
                                      const le_step_plan* plan, float scale, void* out, hipStream_t stream);

/* ------------------------------------------------------------------------
 * (2)+(3) The scatter and the attention of a step in one call.
 * Equals le_kv_cache_write(k_new, v_new, new_dtype, <plan slots>, k_cache,
 * v_cache, kv_dtype, n_tokens, kv_heads*head_dim, num_cache_blocks*block_size)
 * followed by le_ragged_paged_attention on the same plan (the reference's
 * launch_store_kv + attention launch, cuda_model.cu:368-377). When every
 * sequence has one row in the step (decode rows only), the store happens
 * inside the attention launch: the workgroup that owns a row's last context
 * partition writes the row before its first K/V load. Otherwise it is a
 * separate launch first (rows of one prefill chunk read each other's new keys). k_new, v_new: [n_tokens][kv_heads *
 * head_dim] in new_dtype.
 * ------------------------------------------------------------------------ */
int le_ragged_paged_attention_store(const void* q, le_dtype act_dtype, const void* k_new,
                                    const void* v_new, le_dtype new_dtype, void* k_cache,
                                    void* v_cache, le_dtype kv_dtype, int64_t num_cache_blocks,
                                    const le_step_plan* plan, float scale, void* out,
                                    void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------------------------
 * (2)+(3) A layer's attention from its stacked QKV projection rows.
 * Equals le_rope_kv_cache_write(qkv, act_dtype, qkv_row_stride, bias,
 * <plan positions>, <plan slots>, cos_table, sin_table, max_positions, ...,
 * q_scratch, k_cache, v_cache, kv_dtype, num_cache_blocks*block_size)
 * followed by le_ragged_paged_attention(q_scratch, ...) on the same plan,
 * bit for bit (the reference's add_bias + rope + store_kv + attention
 * launches, cuda_model.cu:358-377). When every sequence has one row in the
 * step (decode rows only), bias, RoPE and the K/V store happen inside the
 * attention launch and q_scratch is not touched (it may be null then).
 * qkv: [n_tokens][qkv_row_stride] in act_dtype, q | k | v of each row at
 * element 0, q_heads*head_dim and (q_heads+kv_heads)*head_dim; bias: fp32
 * [(q_heads+2*kv_heads)*head_dim] or null; q_scratch: [n_tokens][q_heads *
 * head_dim] in act_dtype. qkv_row_stride a multiple of 8.
 * ------------------------------------------------------------------------ */
int le_ragged_paged_attention_qkv(const void* qkv, le_dtype act_dtype, int64_t qkv_row_stride,
                                  const float* bias, const float* cos_table, const float* sin_table,
                                  int max_positions, void* k_cache, void* v_cache, le_dtype kv_dtype,
                                  int64_t num_cache_blocks, const le_step_plan* plan, float scale,
                                  void* out, void* q_scratch, void* workspace, size_t workspace_bytes,
                                  hipStream_t stream);

/* le_ragged_paged_attention_qkv with the layer's pre-attention RMSNorm folded
 * into the QKV projection. No counterpart in the reference, whose norm is a
 * launch of its own before the projection (cuda_model.cu:353); for engines
 * that multiply the norm weight into the projection's input columns and
 * project the un-normalised residual stream x. Each row's q, k and v are
 * first multiplied by r = 1/sqrt(mean_j x[t][j]^2 + eps) (fp32, the sum of
 * squares per 16-byte piece and then across a wave), then biased and rounded
 * to act_dtype once, then rotated: the same for the in-launch decode path and
 * the separate rope/store path, so the two stay bit for bit equal. x:
 * [n_tokens][hidden] in act_dtype, 16-byte aligned, hidden a multiple of 8. */
int le_ragged_paged_attention_qkv_rms(const void* qkv, le_dtype act_dtype, int64_t qkv_row_stride,
                                      const float* bias, const void* x, int hidden, float eps,
                                      const float* cos_table, const float* sin_table, int max_positions,
                                      void* k_cache, void* v_cache, le_dtype kv_dtype, int64_t num_cache_blocks,
                                      const le_step_plan* plan, float scale, void* out, void* q_scratch,
                                      void* workspace, size_t workspace_bytes, hipStream_t stream);

/* ------------------------------------------------------------------------
 * The layer ops between the GEMMs and attention, for any element type.
 * The reference launches them one by one (cuda_kernels.h:17-40, called at
 * cuda_model.cu:347-390); the device model here fuses them (residual add
 * with the next norm, bias and RoPE with the cache write), and these entry
 * points let the reference's own call sequence run unchanged (the
 * le_cuda_kernels.h bridge). Arithmetic is fp32 with one rounding to the
 * element type per stored value, as the reference's kernels do. Return 0,
 * a negative le_status for a rejected argument (nothing launched), or the
 * launch's hipError_t.
 * ------------------------------------------------------------------------ */
/* out[t][j] = table[ids[t]][j] (launch_embedding, cuda_kernels.h:17-18). */
int le_embedding(const void* table, le_dtype dtype, const int32_t* ids, void* out, int n_tokens,
                 int hidden, hipStream_t stream);
/* out[r][j] = x[r][j] / sqrt(mean_j x[r][j]^2 + eps) * weight[j], fp32 weight
 * (launch_rmsnorm, cuda_kernels.h:20-23). */
int le_rmsnorm(const void* x, le_dtype dtype, const float* weight, void* out, int rows, int cols,
               float eps, hipStream_t stream);
/* gate[i] = silu(gate[i]) * up[i] in place (launch_silu_mul, cuda_kernels.h:25-26). */
int le_silu_mul(void* gate, const void* up, le_dtype dtype, size_t n, hipStream_t stream);
/* Rotary embedding in place, rotate_half pairing, over x[n_tokens][row_stride]'s
 * first `heads` heads (launch_rope, cuda_kernels.h:28-33). cos/sin tables are
 * [max_pos][head_dim/2] fp32; a token whose position is outside [0, max_pos)
 * is left unchanged (max_pos <= 0: positions are not bounded, as in the
 * reference). */
int le_rope(void* x, le_dtype dtype, const int32_t* positions, const float* cos_table,
            const float* sin_table, int max_pos, int n_tokens, int heads, int head_dim,
            int row_stride, hipStream_t stream);
/* x[i] += y[i] (launch_add_inplace, cuda_kernels.h:35-36). */
int le_add_inplace(void* x, const void* y, le_dtype dtype, size_t n, hipStream_t stream);
/* x[r][c] += bias[c], fp32 bias (launch_add_bias, cuda_kernels.h:38-39). */
int le_add_bias(void* x, le_dtype dtype, const float* bias, int rows, int cols, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* LLM_ENGINE_AMD_H */
