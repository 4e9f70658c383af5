/*
 * llm-engine on MI355X: the reference's launcher signatures, for a drop-in
 * build of its engine.
 *
 * The reference's model code (src/model/cuda/cuda_model.cu:347-410) calls
 * free C++ functions declared in include/engine/cuda_kernels.h:17-64. This
 * header declares all nine with the same names, argument lists and element
 * type (__half, IEEE binary16; fp32 weights, bias and RoPE tables), so those
 * call sites compile unchanged against libllm_engine_amd_bridge.so once the
 * stream type is hipStream_t:
 *
 *   launch_embedding             cuda_kernels.h:17-18   -> le_embedding
 *   launch_rmsnorm               cuda_kernels.h:20-23   -> le_rmsnorm
 *   launch_silu_mul              cuda_kernels.h:25-26   -> le_silu_mul
 *   launch_rope                  cuda_kernels.h:28-33   -> le_rope
 *   launch_add_inplace           cuda_kernels.h:35-36   -> le_add_inplace
 *   launch_add_bias              cuda_kernels.h:38-39   -> le_add_bias
 *   launch_store_kv              cuda_kernels.h:43-45   -> le_kv_cache_write
 *   launch_attention_decode      cuda_kernels.h:50-54   -> le_attention_decode
 *   launch_attention_decode_gqa  cuda_kernels.h:60-64   -> le_attention_decode
 *
 * Each forwards to the C ABI of llm_engine_amd.h with fp16 buffers. Like
 * the reference launchers they return void and throw std::runtime_error on
 * a rejected shape or a failed launch; the reference's no-op cases (zero
 * rows, a null bias) are no-ops here too. Both attention launchers run the
 * same GQA-shared kernel (one K/V read per kv head serves its whole query
 * group), so they give identical results.
 *
 * What the reference signatures cannot carry is registered once, before the
 * first launch (these have no counterpart in the reference):
 *   - the attention workspace (split-K partials and arrival counters), a
 *     device buffer zero-filled once by the caller, at least
 *     le_attention_decode_workspace_size(max_tokens, q_heads, kv_heads,
 *     head_dim) bytes; every launch leaves it zeroed again;
 *   - optionally the cache size in slots (num_blocks * block_size), which
 *     bounds the slots and block ids the kernels accept; without it any
 *     non-negative int32 slot or block id is taken as valid, as the
 *     reference's kernels take them.
 * The registration is process-wide and not thread-safe, like the reference
 * engine, whose single engine thread makes every launch.
 */
#ifndef LE_CUDA_KERNELS_H
#define LE_CUDA_KERNELS_H

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>

namespace engine {

// out[t][j] = table[ids[t]][j] (cuda_kernels.h:17-18).
void launch_embedding(const __half* table, const int32_t* ids, __half* out, int n_tokens, int hidden,
                      hipStream_t stream);

// out[r][j] = x[r][j] * rsqrt(mean(x[r]^2) + eps) * weight[j], fp32 weight (cuda_kernels.h:20-23).
void launch_rmsnorm(const __half* x, const float* weight, __half* out, int rows, int cols, float eps,
                    hipStream_t stream);

// gate[i] = silu(gate[i]) * up[i], in place (cuda_kernels.h:25-26).
void launch_silu_mul(__half* gate, const __half* up, size_t n, hipStream_t stream);

// Rotary embedding in place over x[n_tokens][row_stride], `heads` heads of
// head_dim each, at each token's position (cuda_kernels.h:28-33).
void launch_rope(__half* x, const int* positions, const float* cos_table, const float* sin_table, int n_tokens,
                 int heads, int head_dim, int row_stride, hipStream_t stream);

// x[i] += y[i] (cuda_kernels.h:35-36).
void launch_add_inplace(__half* x, const __half* y, size_t n, hipStream_t stream);

// x[r][c] += bias[c], fp32 bias (cuda_kernels.h:38-39).
void launch_add_bias(__half* x, const float* bias, int rows, int cols, hipStream_t stream);

// Scatter k and v rows into their precomputed cache slots (cuda_kernels.h:43-45).
void launch_store_kv(const __half* k, const __half* v, const int* slots, __half* k_cache, __half* v_cache,
                     int n_tokens, int kv_dim, hipStream_t stream);

// Paged attention over the whole history of each token's own sequence
// (cuda_kernels.h:50-54).
void launch_attention_decode(const __half* q, const __half* k_cache, const __half* v_cache,
                             const int* block_tables, const int* table_offset, const int* token_seq,
                             const int* token_pos, __half* out, int n_tokens, int q_heads, int kv_heads,
                             int head_dim, int block_size, float scale, hipStream_t stream);

// The same computation, one K/V read per kv head (cuda_kernels.h:60-64).
void launch_attention_decode_gqa(const __half* q, const __half* k_cache, const __half* v_cache,
                                 const int* block_tables, const int* table_offset, const int* token_seq,
                                 const int* token_pos, __half* out, int n_tokens, int q_heads, int kv_heads,
                                 int head_dim, int block_size, float scale, hipStream_t stream);

// No counterpart in the reference: the registration described above.
void le_bridge_set_workspace(void* workspace, size_t bytes);
void le_bridge_set_cache_slots(int64_t num_slots);
// Optionally the RoPE tables' length in positions: launch_rope then leaves a
// token whose position is outside [0, max_positions) unchanged. Without it
// positions are not bounded, as in the reference.
void le_bridge_set_rope_positions(int max_positions);

}  // namespace engine

#endif  // LE_CUDA_KERNELS_H
