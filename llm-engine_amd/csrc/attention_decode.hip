// Paged decode attention with GQA-group sharing and split-K (hot-path parts 3, 4).
//
// Computes, for each query row t and query head h (kv head = h / group):
//     out[t][h] = softmax_p( q[t][h] . K[slot(p)][kvh] * scale ) . V[slot(p)][kvh],
//     p in 0..pos[t],  slot(p) = table[p / bs] * bs + p % bs
// Reference: launch_attention_decode_gqa (attention_decode_gqa.cu:87-232) and
// the oracle ref::paged_attention_head (ops.h:87-111).
//
// gfx950 design. The reference runs one block per (token, kv head), which at
// 64 rows x 2 kv heads leaves most of the chip idle; here every row's context
// is cut into partitions and each (row, kv head, partition) is a 256-thread
// workgroup. Each K/V element of a kv head is read from HBM once and serves
// the whole GQA group.
//
//   bf16 cache -> mfma_kernel. The G query heads of the group are the N=16
//     columns of v_mfma_f32_16x16x32_bf16: S^T = K . Q^T takes K rows straight
//     from HBM into A-operand registers (16 keys x 8 dims per lane group), so
//     the score of a key for all G heads costs no vector-ALU work; the softmax
//     runs on the 16 x 16 accumulator (one head per lane column); V is
//     transposed through a wave-private LDS tile and O^T = V^T . P^T reuses the
//     accumulator of P^T directly as the B operand (an MFMA only needs A and B
//     to agree on the order of k inside a lane group). Each wave runs its own
//     online softmax over 64-key tiles; the four waves merge at the end.
//   fp32 cache -> valu_kernel. Exact fp32 products: a K/V row is read with
//     16-byte loads by LPT lanes, q . k partial sums are reduced inside the
//     row's lanes with DPP moves, scores go to LDS, the softmax runs over the
//     whole partition at once, then V is streamed with the probabilities
//     broadcast from LDS.
//
// Split rows are merged inside the same launch: each partition writes its
// unnormalised partial (acc, running max, sum), and the last workgroup of the
// row to arrive (an atomic counter per (row, kv head), reset by that
// workgroup) merges them and writes the output. No second kernel, no extra
// launch gap. Masked positions carry -inf scores and running maxima start at
// -FLT_MAX, so no path computes inf - inf (the reference's sentinel rule,
// attention_decode.cu:81).
#include <float.h>

#include "le_common.h"
#include "le_internal.h"

namespace le {
namespace {

#ifndef LE_DECODE_WAVES
#define LE_DECODE_WAVES 4
#endif
constexpr int kWaves = 4;  // valu_kernel
constexpr int kMfmaWaves = LE_DECODE_WAVES;  // mfma_kernel
constexpr int kMfmaThreads = kMfmaWaves * 64;
constexpr int kThreads = kWaves * kWave;
constexpr int kChunk = 512;   // valu_kernel: scores held in LDS per pass
constexpr int kTile = 64;     // mfma_kernel: keys per wave tile
constexpr int kMaxG = 16;     // heads per kv head the MFMA columns can hold
constexpr int kMergeBatch = 8;       // partial accumulators loaded per batch in the merge
constexpr int kMaxMergeEntries = 1024;  // n_parts * G the merge stages in LDS

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#ifdef LE_PROBE_TIMING
// Diagnostic build only: per-workgroup phase timestamps (100 MHz counter).
__device__ uint64_t g_probe_ts[16384][8];
#define PROBE_TS(k) do { if (threadIdx.x == 0 && blockIdx.y == 0 && blockIdx.x < 16384) \
    g_probe_ts[blockIdx.x][k] = __builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define PROBE_TS(k) do {} while (0)
#endif

struct Work {
  int token, pos, table_off, b_begin, b_end, part, part_begin, n_parts;
  bool valid;
};

// This workgroup's item; valid is false if it has nothing to do (a split past
// the end of a short context in the reference-shaped launch). Returned by
// value so it stays in registers.
__device__ __forceinline__ Work resolve(const DecodeParams& p) {
  if (p.items) {
    const DecodeItem it = p.items[blockIdx.x];
    return Work{it.token, it.pos, it.table_off, it.blk_begin, it.blk_end,
                it.part, it.part_begin, it.n_parts, true};
  }
  const int token = blockIdx.x;
  const int pos = p.token_pos[token];
  const int nb = pos / p.block_size + 1;
  const int ns = min(p.nsplit, nb);
  const int split = blockIdx.z;
  const int b0 = static_cast<int>(static_cast<int64_t>(split) * nb / ns);
  const int b1 = static_cast<int>(static_cast<int64_t>(split + 1) * nb / ns);
  const int pb = token * p.nsplit;
  return Work{token, pos, p.table_offset[p.token_seq[token]], b0, b1,
              ns == 1 ? -1 : pb + split, pb, ns, split < ns};
}

// The new K/V row of a decode row, for kv head kvh, stored by the workgroup
// of the row's last partition (the only one whose keys reach the row's own
// position) before it loads anything from the cache: the scatter of
// le_kv_cache_write (store_kv.cu:20-36) folded into the attention launch.
// One thread per 8-element piece; the caller waits for the stores and
// synchronises the workgroup before its first K/V load, so the row is read
// back from the cache like every other key (no other workgroup reads its
// lines in this launch).
template <typename C>
__device__ __forceinline__ void store_new_row(const DecodeParams& p, const Work& w, int kvh, int hd) {
  if (p.k_new == nullptr || !(w.part < 0 || w.part == w.part_begin + w.n_parts - 1)) return;
  const int pieces = hd / 8;
  const int t = threadIdx.x;
  if (t >= 2 * pieces) return;
  const int64_t slot = p.slots[w.token];
  if (slot < 0 || slot >= p.num_slots) return;
  const int which = t >= pieces;  // 0 = K, 1 = V
  const int c = t - which * pieces;
  const int64_t src = (static_cast<int64_t>(w.token) * p.kv_heads + kvh) * hd + c * 8;
  const int64_t dst = (slot * p.kv_heads + kvh) * hd + c * 8;
  float v[8];
  if (p.new_bf16) {
    elem<bf16_t>::widen(ld16(static_cast<const bf16_t*>(which ? p.v_new : p.k_new) + src), v);
  } else {
    const float* f = static_cast<const float*>(which ? p.v_new : p.k_new) + src;
    elem<float>::widen(ld16(f), v);
    elem<float>::widen(ld16(f + 4), v + 4);
  }
  C* out = static_cast<C*>(const_cast<void*>(which ? p.v_cache : p.k_cache)) + dst;
  if constexpr (sizeof(C) == 2) {
    *reinterpret_cast<uint4*>(out) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                                pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
  } else {
    reinterpret_cast<float4*>(out)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(out)[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
}

// Partials cross workgroups (and XCDs, whose L2s are not coherent with each
// other) through device-coherent accesses: relaxed atomic stores and loads at
// agent scope, which the hardware performs at the coherence point. This avoids
// agent-scope fences, which would write back the whole L2 of the XCD.
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
  return __uint_as_float(__hip_atomic_load(reinterpret_cast<uint32_t*>(const_cast<float*>(p)),
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// Final stage shared by both kernels. fin_acc[g * HD + d] holds the
// workgroup's unnormalised output for head g of the group, fin_ml[g] its
// (max, sum). Writes the output (single partition) or the partial, and in the
// latter case the last arriving workgroup of the row merges all partials.
template <typename ACT, int HD, int NTHR>
__device__ __forceinline__ void finish(const DecodeParams& p, const Work& w, int G, int kvh,
                                       const float* fin_acc, const float2* fin_ml,
                                       float2* merge_ml, float2* merge_w, int* flag) {
  const int tid = threadIdx.x;
  const int64_t head0 = static_cast<int64_t>(w.token) * p.q_heads + kvh * G;
  if (w.part < 0) {
    for (int i = tid; i < G * HD; i += NTHR) {
      const int g = i / HD;
      elem<ACT>::store1(static_cast<ACT*>(p.out) + head0 * HD + i, fin_acc[i] / fin_ml[g].y);
    }
    return;
  }
  const int64_t rec0 = static_cast<int64_t>(w.part) * p.q_heads + kvh * G;
  float* ml = reinterpret_cast<float*>(p.parts.ml);
  for (int i = tid; i < G * HD; i += NTHR) st_dev(p.parts.acc + rec0 * HD + i, fin_acc[i]);
  if (tid < G) {
    st_dev(ml + (rec0 + tid) * 2, fin_ml[tid].x);
    st_dev(ml + (rec0 + tid) * 2 + 1, fin_ml[tid].y);
  }
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores are performed
  __syncthreads();                // ... and every other thread's
  PROBE_TS(4);
  int32_t* counter = p.parts.counters + static_cast<int64_t>(w.token) * p.kv_heads + kvh;
  if (tid == 0)
    *flag = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            w.n_parts - 1;
  __syncthreads();
  PROBE_TS(5);
  if (!*flag) return;
  // Every other partition incremented the counter after its partial was
  // performed, so the coherent loads below see all of them. The loads are
  // issued in batches (all (m, l) pairs at once, then the accumulators
  // kMergeBatch partitions at a time) so the merge costs a few memory
  // latencies, not one per partition.
  const int np = w.n_parts;
  const int64_t rbase = static_cast<int64_t>(w.part_begin) * p.q_heads + kvh * G;
  // Every (m, l) pair and every accumulator value is requested before any is
  // used: one memory round trip for the whole merge (np <= kMergeBatch per
  // batch of accumulators; more partitions take more batches).
  for (int i = tid; i < np * G; i += NTHR) {
    const int j = i / G, g = i - j * G;
    const float* r = ml + (rbase + static_cast<int64_t>(j) * p.q_heads + g) * 2;
    merge_w[i] = make_float2(ld_dev(r), ld_dev(r + 1));  // (m, l) of partition j, head g
  }
  constexpr int kOutPerThread = (kMaxG * HD + NTHR - 1) / NTHR;
  float o[kOutPerThread];
  float v0[kOutPerThread][kMergeBatch];
#pragma unroll
  for (int u = 0; u < kOutPerThread; u++) {
    o[u] = 0.f;
    const int i = min(tid + u * NTHR, G * HD - 1);
#pragma unroll
    for (int b = 0; b < kMergeBatch; b++) {
      const int j = min(b, np - 1);
      v0[u][b] = ld_dev(p.parts.acc + (rbase + static_cast<int64_t>(j) * p.q_heads) * HD + i);
    }
  }
  __syncthreads();
  if (tid < G) {
    float M = -FLT_MAX;
    for (int j = 0; j < np; j++) M = fmaxf(M, merge_w[j * G + tid].x);
    float L = 0.f;
    for (int j = 0; j < np; j++) L += merge_w[j * G + tid].y * exp2f(merge_w[j * G + tid].x - M);
    merge_ml[tid] = make_float2(M, 1.f / L);
  }
  __syncthreads();
  for (int i = tid; i < np * G; i += NTHR) {  // weights exp2(m_j - M) / L
    const int g = i % G;
    merge_w[i].x = exp2f(merge_w[i].x - merge_ml[g].x) * merge_ml[g].y;
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kOutPerThread; u++) {
    const int i = tid + u * NTHR;
    if (i >= G * HD) continue;
    const int g = i / HD;
#pragma unroll
    for (int b = 0; b < kMergeBatch; b++)
      if (b < np) o[u] += v0[u][b] * merge_w[b * G + g].x;
    for (int j0 = kMergeBatch; j0 < np; j0 += kMergeBatch) {
      float v[kMergeBatch];
#pragma unroll
      for (int b = 0; b < kMergeBatch; b++)
        v[b] = ld_dev(p.parts.acc + (rbase + static_cast<int64_t>(min(j0 + b, np - 1)) * p.q_heads) * HD + i);
#pragma unroll
      for (int b = 0; b < kMergeBatch; b++)
        if (j0 + b < np) o[u] += v[b] * merge_w[(j0 + b) * G + g].x;
    }
    elem<ACT>::store1(static_cast<ACT*>(p.out) + head0 * HD + i, o[u]);
  }
  PROBE_TS(6);
  if (tid == 0) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// bf16 cache: MFMA kernel
// ---------------------------------------------------------------------------
template <int HD> struct MfmaLds {
  static constexpr int V_STRIDE = HD * 2 + 16;           // bytes per key row of the V tile
  static constexpr int VT_BYTES = kTile * V_STRIDE;      // per wave
  static constexpr int RED_STRIDE = HD + 4;              // floats per head in the merge area
  static constexpr int RED_BYTES = kMfmaWaves * kMaxG * RED_STRIDE * 4;
  static constexpr int BYTES = (kMfmaWaves * VT_BYTES > RED_BYTES ? kMfmaWaves * VT_BYTES : RED_BYTES);
};

constexpr int kTabCap = 1024;  // block ids of a partition staged in LDS

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

typedef short i16x4 __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16: in each group of 16 lanes, lane i receives 16-bit
// element (i % 4) of the 8-byte chunks addressed by lanes 4j + i/4, j = 0..3.
__device__ __forceinline__ bf16x4 lds_read_tr(const char* p) {
  // C-style cast: the generic LDS pointer becomes an address-space-3 pointer.
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4*)(p));
  return __builtin_bit_cast(bf16x4, v);
}

// One wave's K/V registers for a 64-key tile: this lane's key of each of the
// four 16-key subtiles, KS 16-byte chunks (8 dims) each.
template <int KS> struct TileRegs {
  uint4 k[4][KS], v[4][KS];
  bool ok[4];  // the lane's block id of subtile i was a valid cache block
};

// State the wave carries across tiles.
template <int HD> struct WaveAcc {
  f32x4 acc[HD / 16];
  float m, l;
};

// Issues the tile's 8 * KS 16-byte loads without any branch: a lane whose key
// is past the end (or whose block id is invalid) reads a valid address of the
// cache and is masked afterwards. Branches around loads would make the
// compiler wait for all outstanding loads at every join, serialising them.
// Issues the tile's 8 * KS 16-byte loads without any branch: a lane whose key
// is past the end (or whose block id is invalid) reads a valid address of the
// cache and is masked afterwards. Branches around loads would make the
// compiler wait for all outstanding loads at every join, serialising them.
// Block ids come from the LDS copy of the table (`tab`, indexed from the
// segment's first block), never through a generic pointer: a flat load would
// count against the global-load counter and stall behind the K/V loads.
template <int HD>
__device__ __forceinline__ void load_tile(TileRegs<HD / 32>& r, const bf16_t* kc, const bf16_t* vc,
                                          int key0, int key_end, int kv_stride, int bs_shift,
                                          const int* tab, int tab_base, int col) {
  constexpr int KS = HD / 32;
  const int bs_mask = (1 << bs_shift) - 1;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int key = min(key0 + i * 16 + col, key_end - 1);
    const int bid = tab[(key >> bs_shift) - tab_base];
    r.ok[i] = bid >= 0;  // the staging step marks invalid ids as -1
    const int64_t slot = (static_cast<int64_t>(r.ok[i] ? bid : 0) << bs_shift) + (key & bs_mask);
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
      r.k[i][ks] = ld16_stream(kc + slot * kv_stride + ks * 32);
      r.v[i][ks] = ld16_stream(vc + slot * kv_stride + ks * 32);
    }
  }
}

template <int HD>
__device__ __forceinline__ void compute_tile(WaveAcc<HD>& st, const TileRegs<HD / 32>& r,
                                             const bf16x8* qb, int key0, int key_end,
                                             float scale_log2, char* vt, int col, int grp) {
  using L = MfmaLds<HD>;
  constexpr int KS = HD / 32;
  constexpr int DT = HD / 16;
#ifdef LE_PROBE_NOCOMPUTE
  // Measurement variant: consume the loads, skip the attention arithmetic.
  uint32_t x = 0;
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int ks = 0; ks < KS; ks++) x ^= r.k[i][ks].x ^ r.k[i][ks].w ^ r.v[i][ks].y ^ r.v[i][ks].z;
  st.acc[0][0] += __uint_as_float(x & 0x3fffffff) * 1e-30f;
  st.l += 1.f;
  return;
#endif
  // S^T = K . Q^T: lane holds head `col`, keys key0 + 16i + 4grp + j
  f32x4 s[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    s[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ks++)
      s[i] = mfma16(__builtin_bit_cast(bf16x8, r.k[i][ks]), qb[ks], s[i]);
  }
  float mt = -INFINITY;
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int key = key0 + i * 16 + grp * 4 + j;
      const float v = key < key_end ? s[i][j] * scale_log2 : -INFINITY;
      s[i][j] = v;
      mt = fmaxf(mt, v);
    }
  mt = fmaxf(mt, __shfl_xor(mt, 16, kWave));
  mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
  const float m_new = fmaxf(st.m, mt);
  const float alpha = exp2f(st.m - m_new);
  st.m = m_new;
  float ls = 0.f;
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float e = exp2f(s[i][j] - m_new);
      s[i][j] = e;
      ls += e;
    }
  st.l = st.l * alpha + ls;
#pragma unroll
  for (int d = 0; d < DT; d++) st.acc[d] *= alpha;

  // V rows into this wave's LDS tile, row-major (key rows), with 16-byte
  // stores. A dead key's row is replaced by zeros (its p is 0, but the row
  // read may hold NaNs).
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
      const bool vlive = key0 + i * 16 + col < key_end && r.ok[i];
      *reinterpret_cast<uint4*>(vt + (i * 16 + col) * L::V_STRIDE + (ks * 32 + grp * 8) * 2) =
          vlive ? r.v[i][ks] : make_uint4(0, 0, 0, 0);
    }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // O^T += V^T . P^T over the tile (2 k-steps of 32 keys). The A operand
  // (16 dims x 8 keys per lane group) comes from the row-major tile through
  // the transposing LDS read: lane (col, grp) addresses key row
  // kk*32 + 4*grp + col/4 (then +16) at dims 16*d + 4*(col%4) and receives
  // dim 16*d + col of four keys, the same keys P^T holds for that group.
#pragma unroll
  for (int kk = 0; kk < 2; kk++) {
    bf16x8 pb;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      pb[j] = static_cast<__bf16>(s[2 * kk][j]);
      pb[4 + j] = static_cast<__bf16>(s[2 * kk + 1][j]);
    }
    const char* r_lo = vt + (kk * 32 + grp * 4 + (col >> 2)) * L::V_STRIDE + (col & 3) * 8;
    const char* r_hi = r_lo + 16 * L::V_STRIDE;
#pragma unroll
    for (int d = 0; d < DT; d++) {
      const bf16x4 lo = lds_read_tr(r_lo + d * 32);
      const bf16x4 hi = lds_read_tr(r_hi + d * 32);
      const bf16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      st.acc[d] = mfma16(a, pb, st.acc[d]);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();  // the tile is read before the next one overwrites it
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <typename ACT, int HD>
__global__ __launch_bounds__(kMfmaThreads) void mfma_kernel(DecodeParams p) {
  using L = MfmaLds<HD>;
  constexpr int KS = HD / 32;  // MFMA k-steps over head dims
  constexpr int DT = HD / 16;  // 16-dim output tiles
  // Double-buffered tiles only where the registers allow it.
  constexpr bool kPipe = HD == 64;
  __shared__ __attribute__((aligned(16))) char lds[L::BYTES];
  __shared__ float fin_acc[kMaxG * HD];
  __shared__ float2 fin_ml[kMaxG];
  __shared__ float2 merge_ml[kMaxG];
  __shared__ float2 merge_w[kMaxMergeEntries];
  __shared__ int tab[kTabCap];
  __shared__ int flag;

  PROBE_TS(0);
  // With a plan, the item's block ids sit at a fixed stride: fetch them now,
  // in the same memory round trip as the item itself.
  const bool item_ids = p.items != nullptr && p.item_ids != nullptr && p.ids_stride <= kTabCap;
  constexpr int kIdsPerThread = kTabCap / kMfmaThreads;
  int pre_ids[kIdsPerThread];
  if (item_ids) {
    const int32_t* ids = p.item_ids + static_cast<int64_t>(blockIdx.x) * p.ids_stride;
#pragma unroll
    for (int u = 0; u < kIdsPerThread; u++) {
      const int i = threadIdx.x + u * kMfmaThreads;
      pre_ids[u] = i < p.ids_stride ? ids[i] : -1;
    }
  }
  const Work w = resolve(p);
  if (!w.valid) return;
#ifdef LE_PROBE_TIMING
  if (threadIdx.x == 0 && blockIdx.y == 0 && blockIdx.x < 16384) {
    g_probe_ts[blockIdx.x][4] = __builtin_amdgcn_s_memrealtime() + (w.token & 0) ;
  }
#endif
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int col = lane & 15;   // head of the group (B/C column); key row for A loads
  const int grp = lane >> 4;   // k-group
  const int kvh = blockIdx.y;
  const int G = p.q_heads / p.kv_heads;
  const int bs = p.block_size;
  const int32_t* gtab = p.tables + w.table_off;
  const int kv_stride = p.kv_heads * HD;
  const bf16_t* kc = static_cast<const bf16_t*>(p.k_cache) + kvh * HD + grp * 8;
  const bf16_t* vc = static_cast<const bf16_t*>(p.v_cache) + kvh * HD + grp * 8;
  char* vt = lds + wave * L::VT_BYTES;
  store_new_row<bf16_t>(p, w, kvh, HD);

  // Q^T (B operand): column `col` = head kvh*G + col, 8 dims per k-step.
  bf16x8 qb[KS];
  {
    const bool ok = col < G;
    const ACT* q = static_cast<const ACT*>(p.q) +
                   (static_cast<int64_t>(w.token) * p.q_heads + kvh * G + (ok ? col : 0)) * HD + grp * 8;
#pragma unroll
    for (int ks = 0; ks < KS; ks++)
#pragma unroll
      for (int e = 0; e < 8; e++)
        qb[ks][e] = static_cast<__bf16>(ok ? elem<ACT>::load1(q + ks * 32 + e) : 0.f);
  }

  WaveAcc<HD> st;
#pragma unroll
  for (int d = 0; d < DT; d++) st.acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  st.m = -FLT_MAX;
  st.l = 0.f;
#ifdef LE_PROBE_TIMING
  {
    float qs = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ks++) qs += static_cast<float>(qb[ks][0]);
    if (threadIdx.x == 0 && blockIdx.y == 0 && blockIdx.x < 16384)
      g_probe_ts[blockIdx.x][5] = __builtin_amdgcn_s_memrealtime() + (qs == 12345.f);
    if (threadIdx.x == 0 && blockIdx.y == 0 && blockIdx.x < 16384)
      g_probe_ts[blockIdx.x][6] = __builtin_amdgcn_s_memrealtime() + (pre_ids[0] == 12345);
  }
#endif

  const int bs_shift = __builtin_ctz(bs);  // block sizes are powers of two
  const int stride = kMfmaWaves * kTile;
  // The partition in segments of at most kTabCap blocks: each segment's block
  // ids are staged in LDS (invalid ids as -1), then streamed tile by tile.
  for (int sb0 = w.b_begin; sb0 < w.b_end; sb0 += kTabCap) {
    const int sb1 = min(w.b_end, sb0 + kTabCap);
    __syncthreads();  // the previous segment's table is no longer read
    if (item_ids) {  // one segment: the whole item (ids_stride <= kTabCap)
#pragma unroll
      for (int u = 0; u < kIdsPerThread; u++) {
        const int bid = pre_ids[u];
        tab[tid + u * kMfmaThreads] = (bid >= 0 && bid < p.num_cache_blocks) ? bid : -1;
      }
    } else {
      for (int i = tid; i < sb1 - sb0; i += kMfmaThreads) {
        const int bid = gtab[sb0 + i];
        tab[i] = (bid >= 0 && bid < p.num_cache_blocks) ? bid : -1;
      }
    }
    if (p.k_new != nullptr) __builtin_amdgcn_s_waitcnt(0);  // the new row is stored
    __syncthreads();
    PROBE_TS(1);
    const int key_end = min(sb1 << bs_shift, w.pos + 1);
    int key0 = (sb0 << bs_shift) + wave * kTile;
    if (key0 >= key_end) continue;
    TileRegs<KS> ra;
    load_tile<HD>(ra, kc, vc, key0, key_end, kv_stride, bs_shift, tab, sb0, col);
    if constexpr (kPipe) {
      // The next tile's loads are issued unconditionally (clamped to valid
      // addresses past the end) so every path reaches each compute with the
      // same loads outstanding and the wait before it covers only the tile
      // being computed.
      TileRegs<KS> rb;
      while (true) {
        load_tile<HD>(rb, kc, vc, key0 + stride, key_end, kv_stride, bs_shift, tab, sb0, col);
        compute_tile<HD>(st, ra, qb, key0, key_end, p.scale_log2, vt, col, grp);
        if (key0 + stride >= key_end) break;
        load_tile<HD>(ra, kc, vc, key0 + 2 * stride, key_end, kv_stride, bs_shift, tab, sb0, col);
        compute_tile<HD>(st, rb, qb, key0 + stride, key_end, p.scale_log2, vt, col, grp);
        if (key0 + 2 * stride >= key_end) break;
        key0 += 2 * stride;
      }
    } else {
      while (true) {
        compute_tile<HD>(st, ra, qb, key0, key_end, p.scale_log2, vt, col, grp);
        key0 += stride;
        if (key0 >= key_end) break;
        load_tile<HD>(ra, kc, vc, key0, key_end, kv_stride, bs_shift, tab, sb0, col);
      }
    }
  }

  PROBE_TS(2);
  // ---- merge the four waves ----
  float l_tot = st.l + __shfl_xor(st.l, 16, kWave);
  l_tot += __shfl_xor(l_tot, 32, kWave);
  __syncthreads();  // V^T tiles are dead; reuse the LDS for the merge
  float* red = reinterpret_cast<float*>(lds);  // [wave][head][HD + 4]: acc..., m, l
  if (col < G) {
    float* r = red + (wave * kMaxG + col) * L::RED_STRIDE;
#pragma unroll
    for (int d = 0; d < DT; d++)
      *reinterpret_cast<float4*>(r + d * 16 + grp * 4) =
          make_float4(st.acc[d][0], st.acc[d][1], st.acc[d][2], st.acc[d][3]);
    if (grp == 0) { r[HD] = st.m; r[HD + 1] = l_tot; }
  }
  __syncthreads();
  if (tid < G) {
    float M = -FLT_MAX;
#pragma unroll
    for (int v = 0; v < kMfmaWaves; v++) M = fmaxf(M, red[(v * kMaxG + tid) * L::RED_STRIDE + HD]);
    float Ls = 0.f;
#pragma unroll
    for (int v = 0; v < kMfmaWaves; v++) {
      const float* r = red + (v * kMaxG + tid) * L::RED_STRIDE;
      Ls += r[HD + 1] * exp2f(r[HD] - M);
    }
    fin_ml[tid] = make_float2(M, Ls);
  }
  __syncthreads();
  for (int i = tid; i < G * HD; i += kMfmaThreads) {
    const int g = i / HD, d = i - g * HD;
    const float M = fin_ml[g].x;
    float o = 0.f;
#pragma unroll
    for (int v = 0; v < kMfmaWaves; v++) {
      const float* r = red + (v * kMaxG + g) * L::RED_STRIDE;
      o += r[d] * exp2f(r[HD] - M);
    }
    fin_acc[i] = o;
  }
  __syncthreads();
  PROBE_TS(3);
  finish<ACT, HD, kMfmaThreads>(p, w, G, kvh, fin_acc, fin_ml, merge_ml, merge_w, &flag);
  PROBE_TS(7);
}

// ---------------------------------------------------------------------------
// fp32 cache: vector-ALU kernel (exact fp32 products)
// ---------------------------------------------------------------------------
template <typename ACT, int HD, int G>
__global__ __launch_bounds__(kThreads) void valu_kernel(DecodeParams p) {
  using KV = float;
  constexpr int VEC = elem<KV>::VEC;  // elements per 16-byte load
  constexpr int LPT = HD / VEC;       // lanes per K/V row
  constexpr int TPW = kWave / LPT;    // rows per wave load
  static_assert(LPT <= kWave && (kWave % LPT) == 0, "head_dim too large for one wave");
  static_assert(kChunk * 8 >= kWaves * 8 * HD, "LDS reuse for the cross-wave merge");

  __shared__ float sbuf[kChunk * 8];  // [token][8 heads] scores, then probabilities
  __shared__ float wred[kWaves][8];
  __shared__ float fin_acc[8 * HD];
  __shared__ float2 fin_ml[8];
  __shared__ float2 merge_ml[8];
  __shared__ float2 merge_w[kMaxMergeEntries];
  __shared__ int flag;

  const Work w = resolve(p);
  if (!w.valid) return;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int sub = lane % LPT;
  const int row = lane / LPT;
  const int kvh = blockIdx.y;
  const int bs = p.block_size;
  const int token = w.token;
  const int pos = w.pos;
  const int32_t* table = p.tables + w.table_off;
  const int kv_stride = p.kv_heads * HD;
  const KV* kc = static_cast<const KV*>(p.k_cache) + kvh * HD + sub * VEC;
  const KV* vc = static_cast<const KV*>(p.v_cache) + kvh * HD + sub * VEC;
  if (p.k_new != nullptr) {
    store_new_row<float>(p, w, kvh, HD);
    __builtin_amdgcn_s_waitcnt(0);  // the new row is stored before any wave loads it
    __syncthreads();
  }

  float qf[G][VEC];
  {
    const ACT* q = static_cast<const ACT*>(p.q) +
                   (static_cast<int64_t>(token) * p.q_heads + kvh * G) * HD + sub * VEC;
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
      for (int e = 0; e < VEC; e++) qf[g][e] = elem<ACT>::load1(q + g * HD + e);
  }

  float acc[G][VEC];
  float m_run[G], l_run[G];
#pragma unroll
  for (int g = 0; g < G; g++) {
    m_run[g] = -FLT_MAX;
    l_run[g] = 0.f;
#pragma unroll
    for (int e = 0; e < VEC; e++) acc[g][e] = 0.f;
  }

  const int ntok = (w.b_end - w.b_begin) * bs;
  for (int c0 = 0; c0 < ntok; c0 += kChunk) {
    const int cn = min(kChunk, ntok - c0);
    const int cb0 = w.b_begin + c0 / bs;
    const int cnb = cn / bs;

    // ---- scores: s = (q . k) * scale * log2(e), masked past pos ----
    for (int bi = wave; bi < cnb; bi += kWaves) {
      const int blk = cb0 + bi;
      const int bid = __builtin_amdgcn_readfirstlane(table[blk]);
      const bool ok = bid >= 0 && bid < p.num_cache_blocks;
      const int64_t slot0 = static_cast<int64_t>(ok ? bid : 0) * bs;
      for (int r = 0; r < bs; r += TPW) {
        const int tb = r + row;
        float kf[VEC];
        elem<KV>::widen(ld16_stream(kc + (slot0 + tb) * kv_stride), kf);
        float s[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
          float d = 0.f;
#pragma unroll
          for (int e = 0; e < VEC; e++) d += qf[g][e] * kf[e];
          s[g] = group_sum<LPT>(d);
        }
        const bool live = ok && (blk * bs + tb) <= pos;
        float mine = -INFINITY;
#pragma unroll
        for (int g = 0; g < G; g++)
          if (sub == g) mine = live ? s[g] * p.scale_log2 : -INFINITY;
        if (sub < G) sbuf[(bi * bs + tb) * 8 + sub] = mine;
      }
    }
    __syncthreads();

    // ---- softmax over the chunk: one max and one exp2 per score ----
    float mloc[G];
#pragma unroll
    for (int g = 0; g < G; g++) mloc[g] = -INFINITY;
    for (int t = tid; t < cn; t += kThreads) {
#pragma unroll
      for (int g = 0; g < G; g++) mloc[g] = fmaxf(mloc[g], sbuf[t * 8 + g]);
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
      const float wm = wave_max(mloc[g]);
      if (lane == 0) wred[wave][g] = wm;
    }
    __syncthreads();
    float m_new[G], alpha[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
      float mc = wred[0][g];
#pragma unroll
      for (int v = 1; v < kWaves; v++) mc = fmaxf(mc, wred[v][g]);
      m_new[g] = fmaxf(m_run[g], mc);
      alpha[g] = exp2f(m_run[g] - m_new[g]);
    }
    float lsum[G];
#pragma unroll
    for (int g = 0; g < G; g++) lsum[g] = 0.f;
    for (int t = tid; t < cn; t += kThreads) {
#pragma unroll
      for (int g = 0; g < G; g++) {
        const float e = exp2f(sbuf[t * 8 + g] - m_new[g]);
        sbuf[t * 8 + g] = e;
        lsum[g] += e;
      }
    }
    __syncthreads();  // every thread has read wred's maxima
#pragma unroll
    for (int g = 0; g < G; g++) {
      const float ws = wave_sum(lsum[g]);
      if (lane == 0) wred[wave][g] = ws;
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; g++) {
      float lc = 0.f;
#pragma unroll
      for (int v = 0; v < kWaves; v++) lc += wred[v][g];
      l_run[g] = l_run[g] * alpha[g] + lc;
      m_run[g] = m_new[g];
#pragma unroll
      for (int e = 0; e < VEC; e++) acc[g][e] *= alpha[g];
    }

    // ---- acc += p * v ----
    for (int bi = wave; bi < cnb; bi += kWaves) {
      const int blk = cb0 + bi;
      const int bid = __builtin_amdgcn_readfirstlane(table[blk]);
      const bool ok = bid >= 0 && bid < p.num_cache_blocks;
      if (!ok) continue;  // every score of the block is -inf, so p = 0
      const int64_t slot0 = static_cast<int64_t>(bid) * bs;
      for (int r = 0; r < bs; r += TPW) {
        const int tb = r + row;
        float vf[VEC];
        elem<KV>::widen(ld16_stream(vc + (slot0 + tb) * kv_stride), vf);
        const float4* pr = reinterpret_cast<const float4*>(sbuf + (bi * bs + tb) * 8);
        const float4 p0 = pr[0], p1 = pr[1];
        const float pg[8] = {p0.x, p0.y, p0.z, p0.w, p1.x, p1.y, p1.z, p1.w};
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
          for (int e = 0; e < VEC; e++) acc[g][e] += pg[g] * vf[e];
      }
    }
    __syncthreads();  // sbuf is rewritten by the next chunk
  }

  // ---- merge the TPW rows of each wave (lanes with one `sub`), then the waves ----
#pragma unroll
  for (int g = 0; g < G; g++)
#pragma unroll
    for (int e = 0; e < VEC; e++) {
      float a = acc[g][e];
#pragma unroll
      for (int off = LPT; off < kWave; off <<= 1) {
        if (off == 8) a += dpp::mov<0x128>(a);  // row_ror:8 == lane ^ 8 inside a row
        else a += __shfl_xor(a, off, kWave);
      }
      acc[g][e] = a;
    }
  float* red = sbuf;  // [wave][8][HD]
  if (row == 0) {
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
      for (int e = 0; e < VEC; e++) red[(wave * 8 + g) * HD + sub * VEC + e] = acc[g][e];
  }
#pragma unroll
  for (int g = 0; g < G; g++)
    if (tid == g) fin_ml[g] = make_float2(m_run[g], l_run[g]);
  __syncthreads();
  for (int i = tid; i < G * HD; i += kThreads) {
    const int g = i / HD, d = i % HD;
    float v = red[g * HD + d];
#pragma unroll
    for (int u = 1; u < kWaves; u++) v += red[(u * 8 + g) * HD + d];
    fin_acc[i] = v;
  }
  __syncthreads();
  finish<ACT, HD, kThreads>(p, w, G, kvh, fin_acc, fin_ml, merge_ml, merge_w, &flag);
}

template <typename ACT, int HD, int G>
hipError_t launch_valu(const DecodeParams& p, hipStream_t s) {
  const dim3 grid(p.n_rows, p.kv_heads, p.items ? 1 : p.nsplit);
  valu_kernel<ACT, HD, G><<<grid, kThreads, 0, s>>>(p);
  return hipGetLastError();
}

template <typename ACT, int HD>
hipError_t dispatch_valu(const DecodeParams& p, hipStream_t s) {
  switch (p.q_heads / p.kv_heads) {
    case 1: return launch_valu<ACT, HD, 1>(p, s);
    case 2: return launch_valu<ACT, HD, 2>(p, s);
    case 3: return launch_valu<ACT, HD, 3>(p, s);
    case 4: return launch_valu<ACT, HD, 4>(p, s);
    case 5: return launch_valu<ACT, HD, 5>(p, s);
    case 6: return launch_valu<ACT, HD, 6>(p, s);
    case 7: return launch_valu<ACT, HD, 7>(p, s);
    case 8: return launch_valu<ACT, HD, 8>(p, s);
    default: return hipErrorInvalidValue;
  }
}

template <typename ACT>
hipError_t dispatch(const DecodeParams& p, int kv_bf16, hipStream_t s) {
  const dim3 grid(p.n_rows, p.kv_heads, p.items ? 1 : p.nsplit);
  if (kv_bf16) {
    if (p.head_dim == 64) mfma_kernel<ACT, 64><<<grid, kMfmaThreads, 0, s>>>(p);
    else mfma_kernel<ACT, 128><<<grid, kMfmaThreads, 0, s>>>(p);
    return hipGetLastError();
  }
  return p.head_dim == 64 ? dispatch_valu<ACT, 64>(p, s) : dispatch_valu<ACT, 128>(p, s);
}


}  // namespace

#ifdef LE_PROBE_TIMING
extern "C" int le_probe_timing(void* host, size_t bytes) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_probe_ts), bytes < sizeof(g_probe_ts) ? bytes : sizeof(g_probe_ts)) == hipSuccess ? 0 : 1;
}
extern "C" int le_probe_timing_clear(void) {
  static uint64_t zeros[16384][8];
  return hipMemcpyToSymbol(HIP_SYMBOL(g_probe_ts), zeros, sizeof(zeros)) == hipSuccess ? 0 : 1;
}
#endif

int decode_nsplit(int n_tokens, int kv_heads) {
  const int rows = n_tokens * kv_heads;
  const int target = 2048;  // 8 workgroups per CU on 256 CUs
  int ns = (target + rows - 1) / rows;
  return ns < 1 ? 1 : (ns > 32 ? 32 : ns);
}

hipError_t attention_decode(const DecodeParams& p, int act_bf16, int kv_bf16, hipStream_t s) {
  if (p.n_rows <= 0) return hipSuccess;
  return act_bf16 ? dispatch<bf16_t>(p, kv_bf16, s) : dispatch<float>(p, kv_bf16, s);
}


}  // namespace le
