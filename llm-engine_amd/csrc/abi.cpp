// extern "C" entry points of include/llm_engine_amd.h: argument validation,
// then the launchers in le_internal.h. No exception and no allocation crosses
// this file.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <mutex>
#include <cstring>

#include "le_internal.h"
#include "llm_engine_amd.h"

#ifndef LE_VERSION_STRING
#define LE_VERSION_STRING "llm-engine-amd 0.1 (gfx950)"
#endif

namespace {

int hip_status(hipError_t e) { return e == hipSuccess ? LE_OK : static_cast<int>(e); }

bool valid_dtype(int d) { return d == LE_F32 || d == LE_BF16 || d == LE_F16; }

bool pow2(int x) { return x > 0 && (x & (x - 1)) == 0; }

// Shapes every attention kernel supports.
int check_attention_shape(int q_heads, int kv_heads, int head_dim, int block_size) {
  if (q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || block_size <= 0) return LE_EINVAL;
  if (q_heads % kv_heads != 0) return LE_EINVAL;
  if (q_heads / kv_heads > 8) return LE_EUNSUPPORTED;
  if (head_dim != 64 && head_dim != 128) return LE_EUNSUPPORTED;
  // The score buffer holds 512 positions, a whole number of blocks; a wave
  // load covers up to 8 rows of a block.
  if (!pow2(block_size) || block_size < 8 || block_size > 512) return LE_EUNSUPPORTED;
  return LE_OK;
}

size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// Workspace: a fixed region of arrival counters first, then the partial
// accumulators and (max, sum) pairs. The counter region has the same size for
// every plan, so a workspace reused across steps of different shapes never
// finds an earlier step's partials where this step's counters are: the
// counters are zero at every launch because every launch leaves them zero.
constexpr size_t kCounterRegion = 512 * 1024;  // 65536 (row, kv head) 64-bit counters
size_t counter_bytes(int64_t, int) { return kCounterRegion; }
bool counters_fit(int64_t n_rows, int kv_heads) {
  return static_cast<size_t>(n_rows) * kv_heads * sizeof(uint64_t) <= kCounterRegion;
}

size_t partial_bytes(int64_t n_parts, int64_t n_rows, int q_heads, int kv_heads, int head_dim) {
  return counter_bytes(n_rows, kv_heads) +
         align256(static_cast<size_t>(n_parts) * q_heads * head_dim * sizeof(float)) +
         align256(static_cast<size_t>(n_parts) * q_heads * sizeof(float2));
}

le::PartialLayout carve_partials(void* ws, int64_t n_parts, int64_t n_rows, int q_heads,
                                 int kv_heads, int head_dim) {
  le::PartialLayout L;
  char* b = static_cast<char*>(ws);
  L.counters = reinterpret_cast<unsigned long long*>(b);
  b += counter_bytes(n_rows, kv_heads);
  L.acc = reinterpret_cast<float*>(b);
  b += align256(static_cast<size_t>(n_parts) * q_heads * head_dim * sizeof(float));
  L.ml = reinterpret_cast<float2*>(b);
  return L;
}

}  // namespace

extern "C" {

const char* le_version(void) { return LE_VERSION_STRING; }

const char* le_status_string(int status) {
  switch (status) {
    case LE_OK: return "ok";
    case LE_EINVAL: return "invalid argument";
    case LE_EUNSUPPORTED: return "unsupported shape";
    case LE_ENOSPACE: return "buffer too small";
    case LE_EDEVICE: return "device library failure";
    case LE_ETOOLARGE: return "step needs more than the static scratch holds";
    default: return status > 0 ? hipGetErrorString(static_cast<hipError_t>(status)) : "unknown";
  }
}

int le_kv_cache_write(const void* k, const void* v, le_dtype src_dtype,
                      const int32_t* slot_mapping, void* k_cache, void* v_cache,
                      le_dtype cache_dtype, int n_tokens, int kv_dim, int64_t num_slots,
                      hipStream_t stream) {
  if (n_tokens < 0 || kv_dim <= 0 || num_slots < 0) return LE_EINVAL;
  if (!valid_dtype(src_dtype) || !valid_dtype(cache_dtype)) return LE_EINVAL;
  if (kv_dim % 8 != 0) return LE_EUNSUPPORTED;
  if (n_tokens == 0) return LE_OK;  // the reference returns early on an empty grid
  if (!k || !v || !slot_mapping || !k_cache || !v_cache) return LE_EINVAL;
  return hip_status(le::kv_cache_write(k, v, src_dtype, slot_mapping, k_cache, v_cache, cache_dtype, n_tokens,
                                       kv_dim, num_slots, stream));
}

int le_rope_kv_cache_write(const void* qkv, le_dtype act_dtype, int64_t qkv_row_stride,
                           const float* bias, const int32_t* positions,
                           const int32_t* slot_mapping, const float* cos_table,
                           const float* sin_table, int max_positions, int n_tokens, int q_heads,
                           int kv_heads, int head_dim, void* q_out, void* k_cache, void* v_cache,
                           le_dtype cache_dtype, int64_t num_slots, hipStream_t stream) {
  if (n_tokens < 0 || q_heads <= 0 || kv_heads <= 0 || head_dim <= 0 || num_slots < 0 ||
      max_positions <= 0)
    return LE_EINVAL;
  if (!valid_dtype(act_dtype) || !valid_dtype(cache_dtype)) return LE_EINVAL;
  if (head_dim % 8 != 0) return LE_EUNSUPPORTED;
  if (qkv_row_stride < static_cast<int64_t>(q_heads + 2 * kv_heads) * head_dim) return LE_EINVAL;
  if (qkv_row_stride % 8 != 0) return LE_EUNSUPPORTED;  // 16-byte vector rows
  if (n_tokens == 0) return LE_OK;
  if (!qkv || !positions || !slot_mapping || !cos_table || !sin_table || !q_out || !k_cache ||
      !v_cache)
    return LE_EINVAL;
  return hip_status(le::rope_kv_cache_write(qkv, act_dtype, qkv_row_stride, bias, positions, slot_mapping,
                                            cos_table, sin_table, max_positions, n_tokens, q_heads, kv_heads,
                                            head_dim, q_out, k_cache, v_cache, cache_dtype, num_slots, stream));
}

size_t le_attention_decode_workspace_size(int n_tokens, int q_heads, int kv_heads, int head_dim) {
  if (n_tokens <= 0 || q_heads <= 0 || kv_heads <= 0 || head_dim <= 0) return 0;
  const int ns = le::decode_nsplit(n_tokens, kv_heads);
  return partial_bytes(static_cast<int64_t>(n_tokens) * ns, n_tokens, q_heads, kv_heads, head_dim);
}

int le_attention_decode(const void* q, le_dtype act_dtype, const void* k_cache,
                        const void* v_cache, le_dtype kv_dtype, const int32_t* block_tables,
                        const int32_t* table_offset, const int32_t* token_seq,
                        const int32_t* token_pos, void* out, int n_tokens, int q_heads,
                        int kv_heads, int head_dim, int block_size, float scale,
                        int64_t num_cache_blocks, void* workspace, size_t workspace_bytes,
                        hipStream_t stream) {
  if (n_tokens < 0 || !valid_dtype(act_dtype) || !valid_dtype(kv_dtype)) return LE_EINVAL;
  if (n_tokens == 0) return LE_OK;
  const int shape = check_attention_shape(q_heads, kv_heads, head_dim, block_size);
  if (shape != LE_OK) return shape;
  if (!q || !k_cache || !v_cache || !block_tables || !table_offset || !token_seq || !token_pos ||
      !out || !std::isfinite(scale) || num_cache_blocks <= 0)
    return LE_EINVAL;
  const size_t need = le_attention_decode_workspace_size(n_tokens, q_heads, kv_heads, head_dim);
  if (!counters_fit(n_tokens, kv_heads)) return LE_EUNSUPPORTED;
  if (!workspace || workspace_bytes < need) return LE_ENOSPACE;

  le::DecodeParams p{};
  p.q = q; p.k_cache = k_cache; p.v_cache = v_cache;
  p.tables = block_tables; p.table_offset = table_offset;
  p.token_seq = token_seq; p.token_pos = token_pos; p.out = out;
  p.nsplit = le::decode_nsplit(n_tokens, kv_heads);
  p.parts = carve_partials(workspace, static_cast<int64_t>(n_tokens) * p.nsplit, n_tokens, q_heads,
                           kv_heads, head_dim);
  p.items = nullptr;
  p.n_rows = n_tokens;
  p.q_heads = q_heads; p.kv_heads = kv_heads; p.head_dim = head_dim; p.block_size = block_size;
  p.scale_log2 = scale * 1.4426950408889634f;
  p.num_cache_blocks = num_cache_blocks;
  // Split rows are merged inside the launch (last-arriving partition).
  const hipError_t e = le::attention_decode(p, act_dtype, kv_dtype, stream);
  return hip_status(e);
}

}  // extern "C"

extern "C" {

size_t le_ragged_workspace_size(const le_step_plan* plan) {
  if (!plan || plan->n_parts <= 0) return 0;
  return partial_bytes(plan->n_parts, plan->n_tokens, plan->cfg.q_heads, plan->cfg.kv_heads,
                       plan->cfg.head_dim);
}

}  // extern "C"

namespace {

// A decode step's q and new K/V rows taken straight from the stacked QKV
// projection (bias and RoPE applied inside the attention launch).
struct RopeRows {
  int64_t row_stride;
  const float* bias;
  const float* cos_t;
  const float* sin_t;
  int max_pos;
  const void* rms_x;  // the folded pre-attention RMSNorm's residual stream, or null
  int rms_hidden;
  float rms_eps;
};

// Ragged attention over a packed step; with k_new, the step's new K/V rows are
// stored at the plan's slots first (inside the decode launch on a pure decode
// step, by a scatter launch otherwise).
int ragged_attention(const void* q, le_dtype act_dtype, const void* k_new, const void* v_new,
                     le_dtype new_dtype, const void* k_cache, const void* v_cache, le_dtype kv_dtype,
                     int64_t num_cache_blocks, const le_step_plan* plan, float scale, void* out,
                     void* workspace, size_t workspace_bytes, hipStream_t stream,
                     const RopeRows* rope = nullptr) {
  if (!plan || !valid_dtype(act_dtype) || !valid_dtype(kv_dtype)) return LE_EINVAL;
  if (plan->n_tokens == 0) return LE_OK;
  const le_plan_config& cfg = plan->cfg;
  const int shape = check_attention_shape(cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.block_size);
  if (shape != LE_OK) return shape;
  // A plan routes chunk rows by the cache dtype it was built for.
  if (cfg.kv_dtype != kv_dtype) return LE_EINVAL;
  if (!plan->dev || !q || !k_cache || !v_cache || !out || !std::isfinite(scale) ||
      num_cache_blocks <= 0)
    return LE_EINVAL;
  const size_t need = le_ragged_workspace_size(plan);
  if (need > 0 && !counters_fit(plan->n_tokens, cfg.kv_heads)) return LE_EUNSUPPORTED;
  if (need > 0 && (!workspace || workspace_bytes < need)) return LE_ENOSPACE;

  const char* dev = static_cast<const char*>(plan->dev);
  auto arr = [&](int64_t off) { return reinterpret_cast<const int32_t*>(dev + off); };
  le::PartialLayout parts{};
  if (need > 0)
    parts = carve_partials(workspace, plan->n_parts, plan->n_tokens, cfg.q_heads, cfg.kv_heads,
                           cfg.head_dim);
  const float scale_log2 = scale * 1.4426950408889634f;

  le::DecodeParams d{};
  d.q = q; d.k_cache = k_cache; d.v_cache = v_cache;
  d.tables = arr(plan->off_tables); d.table_offset = arr(plan->off_table_offset);
  d.token_seq = arr(plan->off_token_seq); d.token_pos = arr(plan->off_positions);
  d.out = out; d.parts = parts;
  d.items = reinterpret_cast<const le::DecodeItem*>(dev + plan->off_decode_items);
  d.item_ids = arr(plan->off_decode_ids);
  d.ids_stride = plan->decode_ids_stride;
  d.n_rows = plan->n_decode_items; d.nsplit = 1;
  d.q_heads = cfg.q_heads; d.kv_heads = cfg.kv_heads; d.head_dim = cfg.head_dim;
  d.block_size = cfg.block_size; d.scale_log2 = scale_log2; d.num_cache_blocks = num_cache_blocks;
  d.l2_local = plan->xcd_local && plan->n_parts > 0 && le::xcd_placement_holds(stream);
  // fixed-layout plans hold empty slots, so their item count says nothing
  // about the rounds
  d.wide = cfg.table_capacity == 0 && static_cast<int64_t>(plan->n_decode_items) * cfg.kv_heads >= 512;
  const int64_t num_slots = num_cache_blocks * cfg.block_size;
  hipError_t e = hipSuccess;
  if (k_new) {
    // Inside the launch only if every sequence has a single row in the step:
    // rows of one sequence (a prefill chunk, which an fp32 cache runs as
    // decode rows) read each other's new keys across workgroups.
    if (plan->n_tokens != plan->n_seqs || plan->n_decode_items == 0) {
      e = le::kv_cache_write(k_new, v_new, new_dtype, arr(plan->off_slots), const_cast<void*>(k_cache),
                             const_cast<void*>(v_cache), kv_dtype, plan->n_tokens, cfg.kv_heads * cfg.head_dim,
                             num_slots, stream);
      if (e != hipSuccess) return hip_status(e);
    } else {
      d.k_new = k_new; d.v_new = v_new; d.new_dtype = new_dtype;
      d.slots = arr(plan->off_slots); d.num_slots = num_slots;
      if (rope) {
        d.rope_row_stride = rope->row_stride; d.rope_bias = rope->bias;
        d.rope_cos = rope->cos_t; d.rope_sin = rope->sin_t; d.rope_max_pos = rope->max_pos;
        d.rms_x = rope->rms_x; d.rms_hidden = rope->rms_hidden; d.rms_eps = rope->rms_eps;
      }
    }
  }
  if (rope && !d.k_new) return LE_EINVAL;  // q rows in QKV form need the in-launch path
  if (plan->n_chunk_items == 0)
    return hip_status(le::attention_decode(d, act_dtype, kv_dtype, stream));

  le::ChunkParams c{};
  c.q = q; c.k_cache = k_cache; c.v_cache = v_cache;
  c.tables = d.tables; c.table_offset = d.table_offset; c.token_pos = d.token_pos;
  c.out = out; c.parts = parts;
  c.items = reinterpret_cast<const le::ChunkItem*>(dev + plan->off_chunk_items);
  // chunk items' block ids follow the decode items' at the same stride
  c.item_ids = d.item_ids + static_cast<int64_t>(plan->n_decode_items) * plan->decode_ids_stride;
  c.ids_stride = plan->decode_ids_stride;
  c.n_items = plan->n_chunk_items;
  c.q_heads = cfg.q_heads; c.kv_heads = cfg.kv_heads; c.head_dim = cfg.head_dim;
  c.block_size = cfg.block_size; c.scale_log2 = scale_log2;
  c.num_cache_blocks = num_cache_blocks;
  c.l2_local = d.l2_local;
  // A mixed step is one launch (chunk and decode workgroups in one grid);
  // LE_PLAN_TWO_LAUNCHES runs the two kernels one after the other instead.
  const bool two_launches = (cfg.flags & LE_PLAN_TWO_LAUNCHES) != 0;
  if (plan->n_decode_items > 0 && !two_launches)
    return hip_status(le::attention_ragged(d, c, act_dtype, kv_dtype, stream));
  e = le::attention_decode(d, act_dtype, kv_dtype, stream);
  if (e != hipSuccess) return hip_status(e);
  e = le::attention_chunk(c, act_dtype, kv_dtype, stream);
  return hip_status(e);
}

}  // namespace

extern "C" {

int le_ragged_paged_attention(const void* q, le_dtype act_dtype, const void* k_cache,
                              const void* v_cache, le_dtype kv_dtype, int64_t num_cache_blocks,
                              const le_step_plan* plan, float scale, void* out, void* workspace,
                              size_t workspace_bytes, hipStream_t stream) {
  return ragged_attention(q, act_dtype, nullptr, nullptr, LE_F32, k_cache, v_cache, kv_dtype,
                          num_cache_blocks, plan, scale, out, workspace, workspace_bytes, stream);
}

int le_ragged_paged_attention_store(const void* q, le_dtype act_dtype, const void* k_new,
                                    const void* v_new, le_dtype new_dtype, void* k_cache,
                                    void* v_cache, le_dtype kv_dtype, int64_t num_cache_blocks,
                                    const le_step_plan* plan, float scale, void* out,
                                    void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!k_new || !v_new || !valid_dtype(new_dtype)) return LE_EINVAL;
  if (plan && plan->cfg.head_dim % 8 != 0) return LE_EUNSUPPORTED;
  return ragged_attention(q, act_dtype, k_new, v_new, new_dtype, k_cache, v_cache, kv_dtype,
                          num_cache_blocks, plan, scale, out, workspace, workspace_bytes, stream);
}


static int attention_qkv(const void* qkv, le_dtype act_dtype, int64_t qkv_row_stride,
                                  const float* bias, const float* cos_table, const float* sin_table,
                                  int max_positions, void* k_cache, void* v_cache, le_dtype kv_dtype,
                                  int64_t num_cache_blocks, const le_step_plan* plan, float scale,
                                  void* out, void* q_scratch, void* workspace, size_t workspace_bytes,
                                  hipStream_t stream, const void* rms_x, int rms_hidden, float rms_eps) {
  if (!plan || !valid_dtype(act_dtype) || !valid_dtype(kv_dtype) || max_positions <= 0)
    return LE_EINVAL;
  if (plan->n_tokens == 0) return LE_OK;
  const le_plan_config& cfg = plan->cfg;
  const int shape = check_attention_shape(cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.block_size);
  if (shape != LE_OK) return shape;
  if (cfg.head_dim % 16 != 0) return LE_EUNSUPPORTED;  // both halves of a head in 8-element pieces
  const int qd = cfg.q_heads * cfg.head_dim, kvd = cfg.kv_heads * cfg.head_dim;
  if (qkv_row_stride < static_cast<int64_t>(qd) + 2 * kvd) return LE_EINVAL;
  if (qkv_row_stride % 8 != 0) return LE_EUNSUPPORTED;  // 16-byte vector rows
  if (!qkv || !cos_table || !sin_table || !plan->dev) return LE_EINVAL;
  const size_t esz = act_dtype == LE_F32 ? 4 : 2;
  const char* row0 = static_cast<const char*>(qkv);
  const void* k_new = row0 + qd * esz;
  const void* v_new = row0 + (static_cast<int64_t>(qd) + kvd) * esz;
  if (plan->n_tokens == plan->n_seqs && plan->n_chunk_items == 0 && plan->n_decode_items > 0) {
    // decode rows only: bias, RoPE and the store inside the attention launch
    RopeRows r{qkv_row_stride, bias, cos_table, sin_table, max_positions, rms_x, rms_hidden, rms_eps};
    return ragged_attention(qkv, act_dtype, k_new, v_new, act_dtype, k_cache, v_cache, kv_dtype,
                            num_cache_blocks, plan, scale, out, workspace, workspace_bytes, stream, &r);
  }
  if (!q_scratch || !k_cache || !v_cache) return LE_EINVAL;
  const char* dev = static_cast<const char*>(plan->dev);
  const int32_t* positions = reinterpret_cast<const int32_t*>(dev + plan->off_positions);
  const int32_t* slots = reinterpret_cast<const int32_t*>(dev + plan->off_slots);
  const hipError_t e = le::rope_kv_cache_write(
      qkv, act_dtype, qkv_row_stride, bias, positions, slots, cos_table, sin_table, max_positions, plan->n_tokens,
      cfg.q_heads, cfg.kv_heads, cfg.head_dim, q_scratch, k_cache, v_cache, kv_dtype,
      num_cache_blocks * cfg.block_size, stream, rms_x, rms_hidden, rms_eps);
  if (e != hipSuccess) return hip_status(e);
  return ragged_attention(q_scratch, act_dtype, nullptr, nullptr, LE_F32, k_cache, v_cache, kv_dtype,
                          num_cache_blocks, plan, scale, out, workspace, workspace_bytes, stream, nullptr);
}


int le_ragged_paged_attention_qkv(const void* qkv, le_dtype act_dtype, int64_t qkv_row_stride,
                                  const float* bias, const float* cos_table, const float* sin_table,
                                  int max_positions, void* k_cache, void* v_cache, le_dtype kv_dtype,
                                  int64_t num_cache_blocks, const le_step_plan* plan, float scale,
                                  void* out, void* q_scratch, void* workspace, size_t workspace_bytes,
                                  hipStream_t stream) {
  return attention_qkv(qkv, act_dtype, qkv_row_stride, bias, cos_table, sin_table, max_positions, k_cache, v_cache,
                       kv_dtype, num_cache_blocks, plan, scale, out, q_scratch, workspace, workspace_bytes, stream,
                       nullptr, 0, 0.f);
}

int le_ragged_paged_attention_qkv_rms(const void* qkv, le_dtype act_dtype, int64_t qkv_row_stride,
                                      const float* bias, const void* x, int hidden, float eps,
                                      const float* cos_table, const float* sin_table, int max_positions,
                                      void* k_cache, void* v_cache, le_dtype kv_dtype, int64_t num_cache_blocks,
                                      const le_step_plan* plan, float scale, void* out, void* q_scratch,
                                      void* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!x || hidden <= 0 || !(eps >= 0.f) || !std::isfinite(eps)) return LE_EINVAL;
  if (hidden % 8 != 0 || (reinterpret_cast<uintptr_t>(x) & 15) != 0) return LE_EUNSUPPORTED;  // 16-byte pieces
  return attention_qkv(qkv, act_dtype, qkv_row_stride, bias, cos_table, sin_table, max_positions, k_cache, v_cache,
                       kv_dtype, num_cache_blocks, plan, scale, out, q_scratch, workspace, workspace_bytes, stream, x,
                       hidden, eps);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// le_ragged_paged_attention_noalloc: the ragged attention with its workspace
// in a static device array instead of a caller buffer, for callers that
// cannot allocate. `scratch` is a host-side stand-in for the array in host
// code: its device address comes from hipGetSymbolAddress, once per device,
// and only that address is passed to kernels.
namespace {

constexpr size_t kScratchBytes = size_t{32} << 20;  // 32 MiB per GPU, held until the process ends
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxScratchDevices];  // device address of `scratch`, per device
std::mutex g_scratch_mu;

__global__ void fill_zero_kernel(uint4* p, size_t n16) {
  for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < n16;
       i += static_cast<size_t>(gridDim.x) * blockDim.x)
    p[i] = make_uint4(0, 0, 0, 0);
}

// The current device's address of `scratch`. On the first call on a device
// its arrival counters are cleared with a fill kernel on `stream` (a fill
// kernel, not a memset, so a graph that captures the first call replays
// correctly); every launch leaves them at zero after that.
int scratch_for_device(hipStream_t stream, void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) return LE_EINVAL;
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return static_cast<int>(e);
      fill_zero_kernel<<<64, 256, 0, stream>>>(static_cast<uint4*>(p), kCounterRegion / 16);
      const hipError_t f = hipGetLastError();
      if (f != hipSuccess) return static_cast<int>(f);
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return LE_OK;
}

}  // namespace

extern "C" {

size_t le_noalloc_scratch_bytes(void) { return kScratchBytes; }

int le_ragged_paged_attention_noalloc(const void* q, le_dtype act_dtype, const void* k_cache,
                                      const void* v_cache, le_dtype kv_dtype, int64_t num_cache_blocks,
                                      const le_step_plan* plan, float scale, void* out, hipStream_t stream) {
  if (!plan) return LE_EINVAL;
  if (plan->n_tokens == 0) return LE_OK;
  const size_t need = le_ragged_workspace_size(plan);
  if (need > kScratchBytes) return LE_ETOOLARGE;
  void* ws = nullptr;
  if (need > 0) {
    const int st = scratch_for_device(stream, &ws);
    if (st != LE_OK) return st;
  }
  return ragged_attention(q, act_dtype, nullptr, nullptr, LE_F32, k_cache, v_cache, kv_dtype, num_cache_blocks,
                          plan, scale, out, ws, need > 0 ? kScratchBytes : 0, stream);
}

}  // extern "C"
