// The reference's launcher signatures over the C ABI (le_cuda_kernels.h).
// Host code only: every launch is the library's own (libllm_engine_amd.so).
#include "le_cuda_kernels.h"

#include <stdexcept>
#include <string>

#include "llm_engine_amd.h"

namespace engine {
namespace {

struct Registration {
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
  int64_t num_slots = 0;  // 0: not registered
  int rope_positions = 0;  // 0: not registered
};
Registration g_reg;

// Without a registered cache size, any non-negative int32 slot is accepted.
constexpr int64_t kUnboundedSlots = int64_t{1} << 31;

void check(const char* fn, int status) {
  if (status != LE_OK) throw std::runtime_error(std::string(fn) + ": " + le_status_string(status));
}

void attention(const char* fn, const __half* q, const __half* k_cache, const __half* v_cache,
               const int* block_tables, const int* table_offset, const int* token_seq, const int* token_pos,
               __half* out, int n_tokens, int q_heads, int kv_heads, int head_dim, int block_size, float scale,
               hipStream_t stream) {
  if (block_size <= 0) check(fn, LE_EINVAL);
  const int64_t slots = g_reg.num_slots > 0 ? g_reg.num_slots : kUnboundedSlots;
  const int64_t num_blocks = slots / block_size;
  if (n_tokens > 0 && !g_reg.workspace)
    throw std::runtime_error(std::string(fn) + ": no workspace registered (le_bridge_set_workspace)");
  check(fn, le_attention_decode(q, LE_F16, k_cache, v_cache, LE_F16, block_tables, table_offset, token_seq,
                                token_pos, out, n_tokens, q_heads, kv_heads, head_dim, block_size, scale,
                                num_blocks, g_reg.workspace, g_reg.workspace_bytes, stream));
}

}  // namespace

void le_bridge_set_workspace(void* workspace, size_t bytes) {
  g_reg.workspace = workspace;
  g_reg.workspace_bytes = workspace ? bytes : 0;
}

void le_bridge_set_cache_slots(int64_t num_slots) { g_reg.num_slots = num_slots > 0 ? num_slots : 0; }

void le_bridge_set_rope_positions(int max_positions) { g_reg.rope_positions = max_positions > 0 ? max_positions : 0; }

void launch_embedding(const __half* table, const int32_t* ids, __half* out, int n_tokens, int hidden,
                      hipStream_t stream) {
  if (n_tokens <= 0 || hidden <= 0) return;  // as embedding.cu:27
  check("launch_embedding", le_embedding(table, LE_F16, ids, out, n_tokens, hidden, stream));
}

void launch_rmsnorm(const __half* x, const float* weight, __half* out, int rows, int cols, float eps,
                    hipStream_t stream) {
  if (rows <= 0 || cols <= 0) return;  // as rmsnorm.cu:104
  check("launch_rmsnorm", le_rmsnorm(x, LE_F16, weight, out, rows, cols, eps, stream));
}

void launch_silu_mul(__half* gate, const __half* up, size_t n, hipStream_t stream) {
  if (n == 0) return;
  check("launch_silu_mul", le_silu_mul(gate, up, LE_F16, n, stream));
}

void launch_rope(__half* x, const int* positions, const float* cos_table, const float* sin_table, int n_tokens,
                 int heads, int head_dim, int row_stride, hipStream_t stream) {
  if (n_tokens <= 0 || heads <= 0 || head_dim <= 0) return;  // as rope.cu:56
  check("launch_rope", le_rope(x, LE_F16, positions, cos_table, sin_table, g_reg.rope_positions, n_tokens, heads,
                               head_dim, row_stride, stream));
}

void launch_add_inplace(__half* x, const __half* y, size_t n, hipStream_t stream) {
  if (n == 0) return;
  check("launch_add_inplace", le_add_inplace(x, y, LE_F16, n, stream));
}

void launch_add_bias(__half* x, const float* bias, int rows, int cols, hipStream_t stream) {
  if (rows <= 0 || cols <= 0 || bias == nullptr) return;  // as elementwise.cu:41 (Llama has no bias)
  check("launch_add_bias", le_add_bias(x, LE_F16, bias, rows, cols, stream));
}

void launch_store_kv(const __half* k, const __half* v, const int* slots, __half* k_cache, __half* v_cache,
                     int n_tokens, int kv_dim, hipStream_t stream) {
  const int64_t num_slots = g_reg.num_slots > 0 ? g_reg.num_slots : kUnboundedSlots;
  check("launch_store_kv", le_kv_cache_write(k, v, LE_F16, slots, k_cache, v_cache, LE_F16, n_tokens, kv_dim,
                                             num_slots, stream));
}

void launch_attention_decode(const __half* q, const __half* k_cache, const __half* v_cache,
                             const int* block_tables, const int* table_offset, const int* token_seq,
                             const int* token_pos, __half* out, int n_tokens, int q_heads, int kv_heads,
                             int head_dim, int block_size, float scale, hipStream_t stream) {
  attention("launch_attention_decode", q, k_cache, v_cache, block_tables, table_offset, token_seq, token_pos, out,
            n_tokens, q_heads, kv_heads, head_dim, block_size, scale, stream);
}

void launch_attention_decode_gqa(const __half* q, const __half* k_cache, const __half* v_cache,
                                 const int* block_tables, const int* table_offset, const int* token_seq,
                                 const int* token_pos, __half* out, int n_tokens, int q_heads, int kv_heads,
                                 int head_dim, int block_size, float scale, hipStream_t stream) {
  attention("launch_attention_decode_gqa", q, k_cache, v_cache, block_tables, table_offset, token_seq, token_pos,
            out, n_tokens, q_heads, kv_heads, head_dim, block_size, scale, stream);
}

}  // namespace engine
