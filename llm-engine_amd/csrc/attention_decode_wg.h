#pragma once
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
// is cut into partitions and each (row, kv head, partition) is a workgroup of
// NW waves (decode_wg below: four in the decode kernel, attention_decode.hip;
// eight in the fused ragged kernel, attention_ragged.hip). Each K/V element of
// a kv head is read from HBM once and serves the whole GQA group.
//
//   decode_wg, templated on the cache element type. The G query heads of
//     the group are the N = 16 columns of the MFMA: S^T = K . Q^T takes K rows
//     straight from HBM into A-operand registers, so the score of a key for
//     all G heads costs no vector-ALU work; the softmax runs on the 16 x 16
//     accumulator (one head per lane column); V is staged in a wave-private
//     LDS tile and O^T = V^T . P^T reuses the accumulator of P^T directly as
//     the B operand (an MFMA only needs A and B to agree on the order of k
//     inside a lane group). Each wave runs its own online softmax over its
//     tiles; the waves merge at the end.
//       bf16 / fp16 cache: 64-key tiles on v_mfma_f32_16x16x32_bf16 / _f16,
//       V^T read with the transposing ds_read_b64_tr_b16.
//       fp32 cache: 32-key tiles on v_mfma_f32_16x16x4_f32 (exact fp32
//       products), V^T read as single floats of the row-major tile.
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
namespace dec {
namespace {

constexpr int kTile = 64;     // 16-bit tiles: keys per wave tile
constexpr int kMaxG = 16;     // heads per kv head the MFMA columns can hold
constexpr int kMergeBatch = 8;       // partial accumulators loaded per batch in the merge



struct Work {
  int token, pos, table_off, b_begin, b_end, part, part_begin, n_parts;
  bool valid;
};

// This workgroup's item; valid is false if it has nothing to do (a split past
// the end of a short context in the reference-shaped launch). Returned by
// value so it stays in registers.
__device__ __forceinline__ Work resolve(const DecodeParams& p, int bx, int bz) {
  if (p.items) {
    const DecodeItem it = p.items[bx];
    return Work{it.token, it.pos, it.table_off, it.blk_begin, it.blk_end,
                it.part, it.part_begin, it.n_parts, it.n_parts > 0};  // n_parts 0: padding
  }
  const int token = bx;
  const int pos = p.token_pos[token];
  const int nb = pos / p.block_size + 1;
  const int ns = min(p.nsplit, nb);
  const int split = bz;
  const int b0 = static_cast<int>(static_cast<int64_t>(split) * nb / ns);
  const int b1 = static_cast<int>(static_cast<int64_t>(split + 1) * nb / ns);
  const int pb = token * p.nsplit;
  return Work{token, pos, p.table_offset[p.token_seq[token]], b0, b1,
              ns == 1 ? -1 : pb + split, pb, ns, split < ns};
}

// ---- Rows straight from the stacked QKV projection ----
// The folded pre-attention RMSNorm's row scale r = 1/sqrt(mean(x^2) + eps),
// formed lazily (the decode kernel's folded-norm instantiation): issue() requests the wave's 16-byte pieces of the row of x
// (up to kHeld per lane, held in registers), and get(), called by every lane
// of the wave, reduces them the first time. The loads of the q, k and v rows
// are issued between the two, so the reduction's wait covers only the x
// loads, which are older (loads complete in order). Same per-lane order and
// wave reduction as row_rms_scale, which rope_kv_write_kernel uses: the same
// value. Rows longer than kHeld pieces per lane take row_rms_scale at get().
template <typename ACT> struct RowScale {
  static constexpr int V = 16 / static_cast<int>(sizeof(ACT));
  static constexpr int kHeld = 8;
  const ACT* x = nullptr;  // null: no folded norm, r = 1
  int hidden = 0;
  float eps = 0.f;
  bool done = false;
  float r = 1.f;
  uint4 raw[kHeld];
  __device__ __forceinline__ bool held() const { return hidden <= kHeld * kWave * V; }
  __device__ __forceinline__ void issue() {
    if (!x || !held()) return;
    const int lane = threadIdx.x & (kWave - 1);
    const int last = hidden / V - 1;
#pragma unroll
    for (int i = 0; i < kHeld; i++)
      if (i * kWave * V < hidden) raw[i] = ld16(x + min(lane + i * kWave, last) * V);
  }
  __device__ __forceinline__ float get() {
    if (!x) return 1.f;
    if (!done) {
      if (held()) {
        const int lane = threadIdx.x & (kWave - 1);
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < kHeld; i++) {
          if (i * kWave * V >= hidden) break;
          if ((lane + i * kWave) * V < hidden) {
            float v[8];
            if constexpr (V == 8) {
              elem<ACT>::widen(raw[i], v);
            } else {
              elem<float>::widen(raw[i], v);
            }
#pragma unroll
            for (int e = 0; e < V; e++) ss += v[e] * v[e];
          }
        }
        ss = wave_sum(ss);
        r = 1.0f / sqrtf(ss / hidden + eps);
      } else {
        r = row_rms_scale(x, hidden, eps);
      }
      done = true;
    }
    return r;
  }
};

// Dims [d0, d0 + 8) of one head after bias and rotate_half RoPE (rope.cu:53,
// ops.h:55-66): head is the head's first element in the row, hb its bias (or
// null), cs/sn the position's cos/sin rows. The operations and their order
// are those of rope_kv_write_kernel (bias added and rounded to the activation
// type; a*c - b*s and b*c + a*s without contraction), so q and k are
// bit-identical to that kernel's. d0 is a multiple of 8 and half of head_dim
// a multiple of 8, so the eight dims sit on one side of the rotation.
// scaled: the row is the projection of the un-normalised residual stream
// (the RMSNorm folded into the projection), so each element is first
// multiplied by the row's scale rs, then biased, and rounded once; kLazy:
// the scale is sc->get(), read after this piece's loads are issued.
template <typename ACT, bool kLazy = false, typename XS = ACT>
__device__ __forceinline__ void rope8(const ACT* head, const float* hb, int d0, int half, const float* cs,
                                      const float* sn, float* o, bool scaled = false, float rs = 1.f,
                                      RowScale<XS>* sc = nullptr) {
#pragma clang fp contract(off)
  const bool lo = d0 < half;
  const int dp = lo ? d0 + half : d0 - half;  // the partner dims
  float own[8], oth[8], c[8], s[8];
  elem<ACT>::load8(head + d0, own);
  elem<ACT>::load8(head + dp, oth);
  elem<float>::load8(cs + (lo ? d0 : dp), c);
  elem<float>::load8(sn + (lo ? d0 : dp), s);
  if constexpr (kLazy) {
    scaled = true;
    rs = sc->get();
  }
  if (scaled) {
#pragma unroll
    for (int e = 0; e < 8; e++) {
      own[e] = elem<ACT>::round(hb ? own[e] * rs + hb[d0 + e] : own[e] * rs);
      oth[e] = elem<ACT>::round(hb ? oth[e] * rs + hb[dp + e] : oth[e] * rs);
    }
  } else if (hb) {
#pragma unroll
    for (int e = 0; e < 8; e++) {
      own[e] = elem<ACT>::round(own[e] + hb[d0 + e]);
      oth[e] = elem<ACT>::round(oth[e] + hb[dp + e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const float x = own[e] * c[e];
    const float y = oth[e] * s[e];
    o[e] = lo ? x - y : x + y;
  }
}

// Where load_q reads the query: a q row as attention takes it, or the q part
// of a stacked QKV row, biased and rotated on the way in.
template <typename ACT> struct QRow {
  const ACT* row;
  __device__ __forceinline__ void piece8(int d0, float* o) const { elem<ACT>::load8(row + d0, o); }
};
template <typename ACT, bool kLazy = false> struct QRope {
  const ACT* head;
  const float* hb;
  const float* cs;
  const float* sn;
  int half;
  bool scaled;
  float rs;
  RowScale<ACT>* sc;  // kLazy: the lazily formed row scale (rs and scaled unused)
  // rounded to the activation type, as the separately rotated q is stored
  __device__ __forceinline__ void piece8(int d0, float* o) const {
    rope8<ACT, kLazy>(head, hb, d0, half, cs, sn, o, scaled, rs, sc);
#pragma unroll
    for (int e = 0; e < 8; e++) o[e] = elem<ACT>::round(o[e]);
  }
};

// The new K/V row of a decode row, for kv head kvh, stored by the workgroup
// of the row's last partition (the only one whose keys reach the row's own
// position) before it loads anything from the cache: the scatter of
// le_kv_cache_write (store_kv.cu:20-36) folded into the attention launch.
// One thread per 8-element piece; the caller waits for the stores and
// synchronises the workgroup before any K/V load issued after it, so those
// read the row back from the cache like every other key (no other workgroup
// reads its lines in this launch). A first tile loaded before the store is
// loaded again in that workgroup if it holds the new row's key.
__device__ __forceinline__ bool stores_new_row(const DecodeParams& p, const Work& w) {
  return p.k_new != nullptr && (w.part < 0 || w.part == w.part_begin + w.n_parts - 1);
}
// kFold: the folded-norm instantiation (rows from the stacked QKV projection
// with the row scale sc), the only one that reads sc.
template <typename C, bool kFold = false, typename ACT = float>
__device__ __forceinline__ void store_new_row(const DecodeParams& p, const Work& w, int kvh, int hd, float rs,
                                              RowScale<ACT>* sc = nullptr) {
  if (!stores_new_row(p, w)) return;
  const int pieces = hd / 8;
  const int t = threadIdx.x;
  if constexpr (kFold) {
    // Folded pre-attention norm (rows from the stacked QKV projection, in the
    // activation type): the whole of wave 0 loads (lanes past the 2 * pieces
    // that store read piece 0 again), so the row scale's wave reduction runs
    // with every lane after the row's loads are issued. Same operations as
    // rope8 and the V branch below with the scale.
    if (t >= kWave) return;
    if (w.pos < 0 || w.pos >= p.rope_max_pos) return;  // as rope_kv_write_kernel
    const int64_t slot = p.slots[w.token];
    const bool on = t < 2 * pieces && slot >= 0 && slot < p.num_slots;
    const int tt = t < 2 * pieces ? t : 0;
    const int which = tt >= pieces;  // 0 = K, 1 = V
    const int c = tt - which * pieces;
    const int half = hd / 2, d0 = c * 8;
    const bool lo = d0 < half;
    const int dp = lo ? d0 + half : d0 - half;
    const ACT* h = static_cast<const ACT*>(which ? p.v_new : p.k_new) +
                   static_cast<int64_t>(w.token) * p.rope_row_stride + kvh * hd;
    const float* hb = p.rope_bias ? p.rope_bias + (p.q_heads + which * p.kv_heads + kvh) * hd : nullptr;
    const int64_t tab = static_cast<int64_t>(w.pos) * half;
    float own[8], oth[8], cs[8], sn[8], v[8];
    elem<ACT>::load8(h + d0, own);
    elem<ACT>::load8(h + dp, oth);
    elem<float>::load8(p.rope_cos + tab + (lo ? d0 : dp), cs);
    elem<float>::load8(p.rope_sin + tab + (lo ? d0 : dp), sn);
    const float rs = sc->get();
    {
#pragma clang fp contract(off)
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const float a = elem<ACT>::round(hb ? own[e] * rs + hb[d0 + e] : own[e] * rs);
        const float b = elem<ACT>::round(hb ? oth[e] * rs + hb[dp + e] : oth[e] * rs);
        const float x = a * cs[e];
        const float y = b * sn[e];
        v[e] = which ? a : (lo ? x - y : x + y);
      }
    }
    if (on) {
      const int64_t dst = (slot * p.kv_heads + kvh) * hd + c * 8;
      elem<C>::store8(static_cast<C*>(const_cast<void*>(which ? p.v_cache : p.k_cache)) + dst, v);
    }
    return;
  }
  if (t >= 2 * pieces) return;
  const int64_t slot = p.slots[w.token];
  if (slot < 0 || slot >= p.num_slots) return;
  const int which = t >= pieces;  // 0 = K, 1 = V
  const int c = t - which * pieces;
  const int64_t src = (static_cast<int64_t>(w.token) * p.kv_heads + kvh) * hd + c * 8;
  const int64_t dst = (slot * p.kv_heads + kvh) * hd + c * 8;
  float v[8];
  if (p.rope_max_pos > 0 && (w.pos < 0 || w.pos >= p.rope_max_pos)) return;  // as rope_kv_write_kernel
  const void* src_rows = which ? p.v_new : p.k_new;
  with_dtype(p.new_dtype, [&](auto tag) {
    using S = decltype(tag);
    if (p.rope_max_pos > 0) {
      // k biased and rotated, v biased, as rope_kv_write_kernel stores them
      const int half = hd / 2;
      const int64_t tab = static_cast<int64_t>(w.pos) * half;
      const S* h = static_cast<const S*>(src_rows) + static_cast<int64_t>(w.token) * p.rope_row_stride + kvh * hd;
      const float* hb = p.rope_bias ? p.rope_bias + (p.q_heads + which * p.kv_heads + kvh) * hd : nullptr;
      const bool scaled = p.rms_x != nullptr;
      if (!which) {
        rope8<S>(h, hb, c * 8, half, p.rope_cos + tab, p.rope_sin + tab, v, scaled, rs);
      } else {
        elem<S>::load8(h + c * 8, v);
        if (scaled) {
#pragma unroll
          for (int e = 0; e < 8; e++) v[e] = elem<S>::round(hb ? v[e] * rs + hb[c * 8 + e] : v[e] * rs);
        } else if (hb) {
#pragma unroll
          for (int e = 0; e < 8; e++) v[e] = elem<S>::round(v[e] + hb[c * 8 + e]);
        }
      }
    } else {
      elem<S>::load8(static_cast<const S*>(src_rows) + src, v);
    }
    return 0;
  });
  elem<C>::store8(static_cast<C*>(const_cast<void*>(which ? p.v_cache : p.k_cache)) + dst, v);
}

// Partials cross workgroups, possibly on different XCDs, whose L2s are not
// coherent with each other: they are stored write-through (the sc1 policy of
// agent-scope relaxed atomics) to the coherence point, and read back with
// loads that miss the CU's L1 and take no stale line from the XCD's L2, so a
// merging workgroup never reads a stale value. With l2_local every partition
// of the row shares one XCD, and plain stores into its L2 are enough (the
// same loads read them there). Agent-scope fences are avoided: they write
// back the whole L2 of the XCD.
__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 ld_dev2(const float* p) {  // 8 bytes, 8-byte aligned
  const uint64_t v = __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<float*>(p)), __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float(static_cast<uint32_t>(v)), __uint_as_float(static_cast<uint32_t>(v >> 32)));
}

// The last arriver's merge of a split row: each thread owns one 16-byte
// piece of the output (4 dims of one head) and, for B partitions at a time,
// requests that piece of each partial together with the head's (m, l) (one
// 8-byte load), then folds them in partition order into a running (max,
// sum) with rescaling. Up to B partitions the merge is one memory round
// trip, with no LDS phase or barrier.
template <typename ACT, int HD, int NTHR, int B>
__device__ __forceinline__ void merge_parts(const DecodeParams& p, __amdgpu_buffer_rsrc_t r, const float* ml,
                                            int64_t rbase, int np, int n4, int64_t head0) {
  for (int c = threadIdx.x; c < n4; c += NTHR) {
    const int g = c * 4 / HD;
    float M = -FLT_MAX, L = 0.f;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    for (int j0 = 0; j0 < np; j0 += B) {
      f32x4 x[B];
      float2 mlj[B];
#pragma unroll
      for (int b = 0; b < B; b++) {
        const int64_t jr = static_cast<int64_t>(min(j0 + b, np - 1)) * p.q_heads;
        x[b] = ld_coherent16(r, static_cast<uint32_t>((jr * HD + c * 4) * 4));
        mlj[b] = ld_dev2(ml + (rbase + jr + g) * 2);
      }
#pragma unroll
      for (int b = 0; b < B; b++)
        if (j0 + b < np) {
          // partition j holds sum_p exp2(s_p - m_j) v_p and l_j = sum_p exp2(s_p - m_j)
          const float m_new = fmaxf(M, mlj[b].x);
          const float a = __builtin_amdgcn_exp2f(M - m_new), e = __builtin_amdgcn_exp2f(mlj[b].x - m_new);
          M = m_new;
          L = L * a + mlj[b].y * e;
          o = o * a + x[b] * e;
        }
    }
    const float inv = 1.f / L;
    ACT* out = static_cast<ACT*>(p.out) + head0 * HD + c * 4;
#pragma unroll
    for (int e = 0; e < 4; e++) elem<ACT>::store1(out + e, o[e] * inv);
  }
}

// Final stage, per 16-byte piece (4 dims of head g): the workgroup's
// unnormalised output o and the head's (m, l). A single-partition row writes
// its normalised output; a split row writes the piece of its partial (head g
// of partition part is record part * q_heads + kvh * G + g: HD fp32
// accumulators, then the (m, l) pairs beside).
template <typename ACT, int HD>
__device__ __forceinline__ void write_piece(const DecodeParams& p, const Work& w, int G, int kvh, int c, f32x4 o,
                                            float M, float Ls) {
  const int g = c * 4 / HD;
  if (w.part < 0) {
    ACT* out = static_cast<ACT*>(p.out) + (static_cast<int64_t>(w.token) * p.q_heads + kvh * G) * HD + c * 4;
    const float inv = 1.f / Ls;
#pragma unroll
    for (int e = 0; e < 4; e++) elem<ACT>::store1(out + e, o[e] * inv);
    return;
  }
  const int64_t rec0 = static_cast<int64_t>(w.part) * p.q_heads + kvh * G;
  float* ml = reinterpret_cast<float*>(p.parts.ml);
  const __amdgpu_buffer_rsrc_t r = coherent_rsrc(p.parts.acc + rec0 * HD);
  const bool first = c * 4 - g * HD == 0;  // the head's first piece also writes (m, l)
  if (p.l2_local) {
    st_l2_16(r, static_cast<uint32_t>(c * 16), o);
    if (first) reinterpret_cast<float2*>(ml)[rec0 + g] = make_float2(M, Ls);
  } else {
    st_coherent16(r, static_cast<uint32_t>(c * 16), o);
    if (first) {
      st_dev(ml + (rec0 + g) * 2, M);
      st_dev(ml + (rec0 + g) * 2 + 1, Ls);
    }
  }
}

// After every piece is written: a split row's partitions arrive on the
// row's counter, and the last to arrive merges all partials.
template <typename ACT, int HD, int NTHR>
__device__ __forceinline__ void arrive_and_merge(const DecodeParams& p, const Work& w, int G, int kvh, int* flag) {
  if (w.part < 0) return;
  const int tid = threadIdx.x;
  const int n4 = G * HD / 4;
  const int64_t head0 = static_cast<int64_t>(w.token) * p.q_heads + kvh * G;
  float* ml = reinterpret_cast<float*>(p.parts.ml);
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores are performed
  __syncthreads();                // ... and every other thread's
  arrival_t* counter = p.parts.counters + static_cast<int64_t>(w.token) * p.kv_heads + kvh;
  if (tid == 0) {
    const arrival_t seen = __hip_atomic_fetch_add(counter, arrival_t{1}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = seen == static_cast<arrival_t>(w.n_parts - 1);
  }
  __syncthreads();
  if (!*flag) return;
  // Every other partition incremented the counter after its partial was
  // performed, so the coherent loads of the merge see all of them.
  const int np = w.n_parts;
  const int64_t rbase = static_cast<int64_t>(w.part_begin) * p.q_heads + kvh * G;
  const __amdgpu_buffer_rsrc_t r = coherent_rsrc(p.parts.acc + rbase * HD);
  // Batches as wide as the row's partition count (up to kMergeBatch), so no
  // load is issued twice.
  if (np <= kMergeBatch / 2) {
    merge_parts<ACT, HD, NTHR, kMergeBatch / 2>(p, r, ml, rbase, np, n4, head0);
  } else {
    merge_parts<ACT, HD, NTHR, kMergeBatch>(p, r, ml, rbase, np, n4, head0);
  }
  if (tid == 0) __hip_atomic_store(counter, arrival_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// 16-bit caches (bf16, fp16): MFMA tile
// ---------------------------------------------------------------------------
template <int HD, int VT_BYTES, int NW> struct MfmaLds {
  static constexpr int RED_STRIDE = HD + 4;              // floats per head in the merge area
  static constexpr int RED_BYTES = NW * kMaxG * RED_STRIDE * 4;
  static constexpr int BYTES = (NW * VT_BYTES > RED_BYTES ? NW * VT_BYTES : RED_BYTES);
};
// bytes per key row of a wave's V tile: the row plus 16 bytes against bank conflicts
template <int HD> constexpr int kVStride16 = HD * 2 + 16;

constexpr int kTabCap = 1024;  // block ids of a partition staged in LDS

// One wave's K/V registers for a 64-key tile. K: this lane's key of each of
// the four 16-key subtiles, KS 16-byte chunks (8 dims) each, in the MFMA
// operand layout. V: 4 * KS 16-byte loads bound for the wave's LDS tile, where
// the layout is free (VLanes).
template <int KS> struct TileRegs {
  uint4 k[4][KS], v[4 * KS];
  uint32_t vok;  // bit j: the block id of V load j was a valid cache block
};

// The key row of the tile and the 16-byte piece of it that this lane moves in
// V load j, for key rows of ROW_BYTES. With WHOLE, each load instruction
// covers whole rows (ROW_BYTES / 16 lanes per row, consecutive rows per load):
// with 128-byte rows that reads 8 whole rows per instruction instead of half
// of each of 16 rows (the K operand layout), config 2 13.2 -> 12.9 us.
// Without it, load j is the K operand layout's: row 16 * (j / KS) + col, piece
// 4 * (j % KS) + group (kept for 256-byte 16-bit rows, where whole rows need
// 16 address computations per tile and the tile no longer fits two waves per
// SIMD).
template <int ROW_BYTES, bool WHOLE, int KS> struct VLanes {
  static constexpr int kLanesPerRow = ROW_BYTES / 16;
  static constexpr int kRowsPerLoad = kWave / kLanesPerRow;
  int a, b;  // WHOLE: first row, piece; else: col, group
  __device__ __forceinline__ VLanes() {
    const int lane = threadIdx.x & (kWave - 1);
    a = WHOLE ? lane / kLanesPerRow : lane & 15;
    b = WHOLE ? lane % kLanesPerRow : lane >> 4;
  }
  __device__ __forceinline__ int row(int j) const { return WHOLE ? j * kRowsPerLoad + a : (j / KS) * 16 + a; }
  __device__ __forceinline__ int piece(int j) const { return WHOLE ? b : (j % KS) * 4 + b; }
};
template <int HD> using VLanes16 = VLanes<HD * 2, HD == 64, HD / 32>;

// State the wave carries across tiles.
template <int HD> struct WaveAcc {
  f32x4 acc[HD / 16];
  float m, l;
};

// Issues the tile's 8 * KS 16-byte loads without any branch: a lane whose key
// is past the end (or whose block id is invalid) reads a valid address of the
// cache and is masked afterwards. Branches around loads would make the
// compiler wait for all outstanding loads at every join, serialising them.
// Block ids come from the LDS copy of the table (`tab`, indexed from the
// segment's first block), never through a generic pointer: a flat load would
// count against the global-load counter and stall behind the K/V loads.
// Online softmax of one tile (log2 domain). s holds the tile's scaled scores
// (-inf for dead keys) in a lane's column, mt their maximum over the column.
// The arguments of exp2 are <= 0, so the raw hardware exp2 (whose results
// below 2^-126 flush to zero) suffices; exp2f wraps a denormal-safe scaling
// around it on every score. The rescale is unconditional: a wave-uniform
// branch around it splits the loop body, and the next tile's loads then no
// longer interleave with this tile's arithmetic (28.6 -> 29.7 us on 64 rows
// x 4096 keys).
template <int NS, int HD>
__device__ __forceinline__ void softmax_tile(WaveAcc<HD>& st, f32x4 (&s)[NS], float mt) {
  const float m_new = fmaxf(st.m, mt);
  const float alpha = __builtin_amdgcn_exp2f(st.m - m_new);
  st.m = m_new;
  float ls = 0.f;
#pragma unroll
  for (int i = 0; i < NS; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const float e = __builtin_amdgcn_exp2f(s[i][j] - m_new);
      s[i][j] = e;
      ls += e;
    }
  st.l = st.l * alpha + ls;
#pragma unroll
  for (int d = 0; d < HD / 16; d++) st.acc[d] *= alpha;
}

template <typename T, int HD>
__device__ __forceinline__ void load_tile(TileRegs<HD / 32>& r, const T* kc, const T* vc,
                                          int key0, int key_end, int kv_stride, int bs_shift,
                                          const int* tab, int tab_base, int col) {
  constexpr int KS = HD / 32;
  const int bs_mask = (1 << bs_shift) - 1;
  const VLanes16<HD> vl;
  // vc points at this lane's K operand dims (group * 8); V loads address
  // their own pieces from the row start
  const T* vrow = vc - (threadIdx.x & (kWave - 1)) / 16 * 8;
  r.vok = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int key = min(key0 + i * 16 + col, key_end - 1);
    const int bid = tab[(key >> bs_shift) - tab_base];
    const bool ok = bid >= 0;  // the staging step marks invalid ids as -1
    const int64_t slot = (static_cast<int64_t>(ok ? bid : 0) << bs_shift) + (key & bs_mask);
#pragma unroll
    for (int ks = 0; ks < KS; ks++) r.k[i][ks] = ld16_stream(kc + slot * kv_stride + ks * 32);
  }
#pragma unroll
  for (int j = 0; j < 4 * KS; j++) {
    const int key = min(key0 + vl.row(j), key_end - 1);
    const int bid = tab[(key >> bs_shift) - tab_base];
    const bool ok = bid >= 0;
    r.vok |= static_cast<uint32_t>(ok) << j;
    const int64_t slot = (static_cast<int64_t>(ok ? bid : 0) << bs_shift) + (key & bs_mask);
    r.v[j] = ld16_stream(vrow + slot * kv_stride + vl.piece(j) * 8);
  }
}

template <typename T, int HD>
__device__ __forceinline__ void compute_tile(WaveAcc<HD>& st, const TileRegs<HD / 32>& r,
                                             const typename mma16<T>::v8* qb, int key0, int key_end,
                                             float scale_log2, char* vt, int col, int grp) {
  using M = mma16<T>;
  constexpr int V_STRIDE = kVStride16<HD>;
  constexpr int KS = HD / 32;
  constexpr int DT = HD / 16;
  // S^T = K . Q^T: lane holds head `col`, keys key0 + 16i + 4grp + j
  f32x4 s[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    s[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ks++)
      s[i] = M::mma(__builtin_bit_cast(typename M::v8, r.k[i][ks]), qb[ks], s[i]);
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
  softmax_tile<4>(st, s, mt);

  // V rows into this wave's LDS tile, row-major (key rows), with 16-byte
  // stores. A dead key's row is replaced by zeros (its p is 0, but the row
  // read may hold NaNs).
  const VLanes16<HD> vl;
#pragma unroll
  for (int j = 0; j < 4 * KS; j++) {
    // a mask, not a select: a select becomes a branch, and the loads it
    // skips count as outstanding at every later join (the loop head then
    // waits for the next tile's loads too)
    const int row = vl.row(j);
    const uint32_t m = 0u - static_cast<uint32_t>(key0 + row < key_end && ((r.vok >> j) & 1u));
    const uint4 v = r.v[j];
    *reinterpret_cast<uint4*>(vt + row * V_STRIDE + vl.piece(j) * 16) = make_uint4(v.x & m, v.y & m, v.z & m, v.w & m);
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
    typename M::v8 pb;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      pb[j] = static_cast<typename M::scalar>(s[2 * kk][j]);
      pb[4 + j] = static_cast<typename M::scalar>(s[2 * kk + 1][j]);
    }
    const char* r_lo = vt + (kk * 32 + grp * 4 + (col >> 2)) * V_STRIDE + (col & 3) * 8;
    const char* r_hi = r_lo + 16 * V_STRIDE;
#pragma unroll
    for (int d = 0; d < DT; d++) {
      const typename M::v4 lo = lds_read_tr16<T>(r_lo + d * 32);
      const typename M::v4 hi = lds_read_tr16<T>(r_hi + d * 32);
      const typename M::v8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      st.acc[d] = M::mma(a, pb, st.acc[d]);
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();  // the tile is read before the next one overwrites it
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Tile operations of the MFMA decode kernel, per cache element type. A tile is
// one wave's kKeys consecutive keys; the kernel around it (item, block ids,
// pipelining, cross-wave and cross-workgroup merge) is shared.
template <typename KV, int HD> struct DecodeTile;

// 16-bit cache of element type T: 64-key tiles on the 16x16x32 MFMA of T (load_tile,
// compute_tile above).
template <typename T, int HD> struct DecodeTile16 {
  static constexpr int kKeys = kTile;
  static constexpr int VT_BYTES = kKeys * kVStride16<HD>;
  static constexpr bool kPipe = HD == 64;  // double-buffered where the registers allow it
  static constexpr bool kEarly = HD == 64;  // first tile issued before the item is read (HD 128: too many registers)
  static constexpr int kLaneElems = 8;     // dims per lane group and k-step
  using Regs = TileRegs<HD / 32>;
  using M = mma16<T>;
  struct QOp { typename M::v8 b[HD / 32]; };
  template <typename Src>
  __device__ __forceinline__ static void load_q(QOp& q, const Src& src, bool ok, int grp) {
    // unconditional 16-byte loads (the row pointer is valid for every
    // lane), selected afterwards: a load under a branch is waited for
    // before the next one is issued
    float f[HD / 32][8];
#pragma unroll
    for (int ks = 0; ks < HD / 32; ks++) src.piece8(grp * 8 + ks * 32, f[ks]);
#pragma unroll
    for (int ks = 0; ks < HD / 32; ks++)
#pragma unroll
      for (int e = 0; e < 8; e++) q.b[ks][e] = static_cast<typename M::scalar>(ok ? f[ks][e] : 0.f);
  }
  __device__ __forceinline__ static const T* lane_base(const void* cache, int kvh, int grp) {
    return static_cast<const T*>(cache) + kvh * HD + grp * 8;
  }
  __device__ __forceinline__ static void load(Regs& r, const T* kc, const T* vc, int key0, int key_end,
                                              int kv_stride, int bs_shift, const int* tab, int tab_base, int col) {
    load_tile<T, HD>(r, kc, vc, key0, key_end, kv_stride, bs_shift, tab, tab_base, col);
  }
  __device__ __forceinline__ static void compute(WaveAcc<HD>& st, const Regs& r, const QOp& q, int key0, int key_end,
                                                 float scale_log2, char* vt, int col, int grp) {
    compute_tile<T, HD>(st, r, q.b, key0, key_end, scale_log2, vt, col, grp);
  }
  // The first tile, addressed without the item: key rel0 + 16i + col of the
  // item reads block ids[rel >> bs_shift] (the plan pads ids with -1 past
  // the item, so those keys read block 0 and are masked by the caller).
  __device__ __forceinline__ static void load_direct(Regs& r, const T* kc, const T* vc, int rel0,
                                                     const int32_t* ids, int n_ids, int bs_shift, int kv_stride,
                                                     int64_t num_blocks, int col) {
    constexpr int KS = HD / 32;
    const int bs_mask = (1 << bs_shift) - 1;
    const VLanes16<HD> vl;
    const T* vrow = vc - (threadIdx.x & (kWave - 1)) / 16 * 8;
    r.vok = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int rel = rel0 + i * 16 + col;
      const int bid = ids[min(rel >> bs_shift, n_ids - 1)];
      const bool ok = bid >= 0 && bid < num_blocks;
      const int64_t slot = (static_cast<int64_t>(ok ? bid : 0) << bs_shift) + (rel & bs_mask);
#pragma unroll
      for (int ks = 0; ks < KS; ks++) r.k[i][ks] = ld16_stream(kc + slot * kv_stride + ks * 32);
    }
#pragma unroll
    for (int j = 0; j < 4 * KS; j++) {
      const int rel = rel0 + vl.row(j);
      const int bid = ids[min(rel >> bs_shift, n_ids - 1)];
      const bool ok = bid >= 0 && bid < num_blocks;
      r.vok |= static_cast<uint32_t>(ok) << j;
      const int64_t slot = (static_cast<int64_t>(ok ? bid : 0) << bs_shift) + (rel & bs_mask);
      r.v[j] = ld16_stream(vrow + slot * kv_stride + vl.piece(j) * 8);
    }
  }
};

template <int HD> struct DecodeTile<bf16_t, HD> : DecodeTile16<bf16_t, HD> {};
template <int HD> struct DecodeTile<f16_t, HD> : DecodeTile16<f16_t, HD> {};

// fp32 cache: 32-key tiles on v_mfma_f32_16x16x4_f32, exact fp32 products.
//   S^T = K . Q^T: lane (col, grp) holds key col of each 16-key subtile with
//   its dims [grp*HD/4, (grp+1)*HD/4) (contiguous, 16-byte loads); k-step j
//   takes dim grp*HD/4 + j from both K (A) and Q^T (B), so the sum over
//   lane groups and steps covers every dim once.
//   O^T += V^T . P^T: k-step j of the product covers keys
//   16*(j/4) + 4*grp + j%4, which are exactly the scores the lane's S^T
//   accumulators hold, so P^T needs no shuffle; the V^T operand reads
//   single floats of the row-major V tile staged in LDS.
template <int HD> struct DecodeTile<float, HD> {
  static constexpr int kKeys = 32;
  static constexpr int kSub = kKeys / 16;   // 16-key subtiles
  static constexpr int kLaneDims = HD / 4;  // dims per lane per key
  static constexpr int kPieces = kLaneDims / 4;  // 16-byte loads per lane per key
  static constexpr int V_STRIDE = HD * 4 + 16;   // bytes per key row of the V tile
  static constexpr int VT_BYTES = kKeys * V_STRIDE;
  static constexpr bool kPipe = HD == 64;
  static constexpr bool kEarly = false;  // measured slower: more registers for no gain
  using VL = VLanes<HD * 4, true, 0>;
  // K in the MFMA operand layout; V as whole key rows for the LDS tile
  struct Regs {
    float4 k[kSub][kPieces], v[kSub * kPieces];
    uint32_t vok;  // bit j: the block id of V load j was a valid cache block
  };
  struct QOp { float q[kLaneDims]; };
  template <typename Src>
  __device__ __forceinline__ static void load_q(QOp& q, const Src& src, bool ok, int grp) {
    float f[kLaneDims];  // unconditional vector loads, as in the bf16 tile
#pragma unroll
    for (int j = 0; j < kLaneDims; j += 8) src.piece8(grp * kLaneDims + j, &f[j]);
#pragma unroll
    for (int j = 0; j < kLaneDims; j++) q.q[j] = ok ? f[j] : 0.f;
  }
  __device__ __forceinline__ static const float* lane_base(const void* cache, int kvh, int grp) {
    return static_cast<const float*>(cache) + kvh * HD + grp * kLaneDims;
  }
  // Branch-free like the bf16 tile: a lane whose key is past the end (or in
  // an invalid block) reads a valid address and is masked afterwards.
  __device__ __forceinline__ static void load(Regs& r, const float* kc, const float* vc, int key0, int key_end,
                                              int kv_stride, int bs_shift, const int* tab, int tab_base, int col) {
    const int bs_mask = (1 << bs_shift) - 1;
    const VL vl;
    const float* vrow = vc - (threadIdx.x & (kWave - 1)) / 16 * kLaneDims + vl.piece(0) * 4;
    r.vok = 0;
#pragma unroll
    for (int i = 0; i < kSub; i++) {
      const int key = min(key0 + i * 16 + col, key_end - 1);
      const int bid = tab[(key >> bs_shift) - tab_base];
      const bool ok = bid >= 0;
      const int64_t slot = (static_cast<int64_t>(ok ? bid : 0) << bs_shift) + (key & bs_mask);
#pragma unroll
      for (int c = 0; c < kPieces; c++) r.k[i][c] = as_float4(ld16_stream(kc + slot * kv_stride + c * 4));
    }
#pragma unroll
    for (int j = 0; j < kSub * kPieces; j++) {
      const int key = min(key0 + vl.row(j), key_end - 1);
      const int bid = tab[(key >> bs_shift) - tab_base];
      const bool ok = bid >= 0;
      r.vok |= static_cast<uint32_t>(ok) << j;
      const int64_t slot = (static_cast<int64_t>(ok ? bid : 0) << bs_shift) + (key & bs_mask);
      r.v[j] = as_float4(ld16_stream(vrow + slot * kv_stride));
    }
  }
  __device__ __forceinline__ static void load_direct(Regs& r, const float* kc, const float* vc, int rel0,
                                                     const int32_t* ids, int n_ids, int bs_shift, int kv_stride,
                                                     int64_t num_blocks, int col) {
    const int bs_mask = (1 << bs_shift) - 1;
    const VL vl;
    const float* vrow = vc - (threadIdx.x & (kWave - 1)) / 16 * kLaneDims + vl.piece(0) * 4;
    r.vok = 0;
#pragma unroll
    for (int i = 0; i < kSub; i++) {
      const int rel = rel0 + i * 16 + col;
      const int bid = ids[min(rel >> bs_shift, n_ids - 1)];
      const bool ok = bid >= 0 && bid < num_blocks;
      const int64_t slot = (static_cast<int64_t>(ok ? bid : 0) << bs_shift) + (rel & bs_mask);
#pragma unroll
      for (int c = 0; c < kPieces; c++) r.k[i][c] = as_float4(ld16_stream(kc + slot * kv_stride + c * 4));
    }
#pragma unroll
    for (int j = 0; j < kSub * kPieces; j++) {
      const int rel = rel0 + vl.row(j);
      const int bid = ids[min(rel >> bs_shift, n_ids - 1)];
      const bool ok = bid >= 0 && bid < num_blocks;
      r.vok |= static_cast<uint32_t>(ok) << j;
      const int64_t slot = (static_cast<int64_t>(ok ? bid : 0) << bs_shift) + (rel & bs_mask);
      r.v[j] = as_float4(ld16_stream(vrow + slot * kv_stride));
    }
  }
  __device__ __forceinline__ static void compute(WaveAcc<HD>& st, const Regs& r, const QOp& q, int key0, int key_end,
                                                 float scale_log2, char* vt, int col, int grp) {
    constexpr int DT = HD / 16;
    // ---- S^T: kSub subtiles of 16 keys x 16 heads ----
    f32x4 s[kSub];
#pragma unroll
    for (int i = 0; i < kSub; i++) {
      s[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < kPieces; c++) {
        const float kv4[4] = {r.k[i][c].x, r.k[i][c].y, r.k[i][c].z, r.k[i][c].w};
#pragma unroll
        for (int e = 0; e < 4; e++) s[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv4[e], q.q[c * 4 + e], s[i], 0, 0, 0);
      }
    }
    float mt = -INFINITY;
#pragma unroll
    for (int i = 0; i < kSub; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int key = key0 + i * 16 + grp * 4 + j;
        const float v = key < key_end ? s[i][j] * scale_log2 : -INFINITY;
        s[i][j] = v;
        mt = fmaxf(mt, v);
      }
    mt = fmaxf(mt, __shfl_xor(mt, 16, kWave));
    mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
    softmax_tile<kSub>(st, s, mt);

    // V rows into this wave's LDS tile (row-major); a dead key's row is zeros.
    const VL vl;
#pragma unroll
    for (int j = 0; j < kSub * kPieces; j++) {
      const int row = vl.row(j);
      const uint32_t m = 0u - static_cast<uint32_t>(key0 + row < key_end && ((r.vok >> j) & 1u));  // as above
      const float4 v = r.v[j];
      *reinterpret_cast<float4*>(vt + row * V_STRIDE + vl.piece(j) * 16) =
          make_float4(__uint_as_float(__float_as_uint(v.x) & m), __uint_as_float(__float_as_uint(v.y) & m),
                      __uint_as_float(__float_as_uint(v.z) & m), __uint_as_float(__float_as_uint(v.w) & m));
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- O^T += V^T . P^T: k-step j covers keys 16*(j/4) + 4*grp + j%4 ----
#pragma unroll
    for (int j = 0; j < kSub * 4; j++) {
      const float pb = s[j >> 2][j & 3];
      const float* vrow = reinterpret_cast<const float*>(vt + (16 * (j >> 2) + 4 * grp + (j & 3)) * V_STRIDE);
#pragma unroll
      for (int d = 0; d < DT; d++) st.acc[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(vrow[d * 16 + col], pb, st.acc[d], 0, 0, 0);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();  // the tile is read before the next one overwrites it
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
};

// LDS of one decode workgroup of NW waves.
template <typename KV, int HD, int NW> struct DecodeSmem {
  using L = MfmaLds<HD, DecodeTile<KV, HD>::VT_BYTES, NW>;
  __attribute__((aligned(16))) char lds[L::BYTES];
  int tab[kTabCap];
  int flag;
};

// One decode workgroup of NW waves: item (or row) bx, kv head by, split bz
// (the reference-shaped launch without a plan). Shared by the decode kernel
// and the fused ragged kernel.
// kFold: rows straight from the stacked QKV projection with the folded
// pre-attention norm (p.rms_x set, p.rope_max_pos > 0), the row scale formed
// lazily behind the row loads; an instantiation of its own, so the code of
// every other path is not shaped by it.
template <typename ACT, typename KV, int HD, int NW, bool kFold = false>
__device__ __forceinline__ void decode_wg(const DecodeParams& p, DecodeSmem<KV, HD, NW>& sm, int bx, int by, int bz) {
  using T = DecodeTile<KV, HD>;
  using L = MfmaLds<HD, T::VT_BYTES, NW>;
  constexpr int kMfmaWaves = NW;
  constexpr int kMfmaThreads = NW * kWave;
  constexpr int DT = HD / 16;  // 16-dim output tiles
  constexpr bool kPipe = T::kPipe;
  char* lds = sm.lds;
  int* tab = sm.tab;
  [[maybe_unused]] const uint64_t t_start = LE_TIM_NOW();

  // With a plan, the item's block ids sit at a fixed stride: fetch them now,
  // in the same memory round trip as the item itself, and issue each wave's
  // first tile straight from them: its addresses need no field of the item.
  const bool item_ids = p.items != nullptr && p.item_ids != nullptr && p.ids_stride <= kTabCap;
  const bool early = T::kEarly && item_ids;
  constexpr int kIdsPerThread = kTabCap / kMfmaThreads;
  int pre_ids[kIdsPerThread];
  const int32_t* ids_row = p.item_ids + static_cast<int64_t>(bx) * p.ids_stride;
  typename T::Regs ra;
  if (item_ids) {
#pragma unroll
    for (int u = 0; u < kIdsPerThread; u++) {
      const int i = threadIdx.x + u * kMfmaThreads;
      pre_ids[u] = i < p.ids_stride ? ids_row[i] : -1;
    }
  }
#ifdef LE_TIMING_RT
  // round-trip probe (measurement builds only; serialises the first loads)
  __builtin_amdgcn_s_waitcnt(0);
  LE_TIM(8, LE_TIM_NOW());
#endif
  if (early) {
    T::load_direct(ra, T::lane_base(p.k_cache, by, threadIdx.x >> 4 & 3),
                   T::lane_base(p.v_cache, by, threadIdx.x >> 4 & 3), (threadIdx.x >> 6) * T::kKeys,
                   ids_row, p.ids_stride, __builtin_ctz(p.block_size), p.kv_heads * HD, p.num_cache_blocks,
                   threadIdx.x & 15);
  }
#ifdef LE_TIMING_RT
  __builtin_amdgcn_s_waitcnt(0);
  LE_TIM(9, LE_TIM_NOW());
#endif
  const Work w = resolve(p, bx, bz);
  if (!w.valid) return;
  LE_TIM(0, t_start);
  LE_TIM(5, LE_TIM_PLACE());
#ifdef LE_TIMING_RT
  LE_TIM(7, 3);  // decode, slots 8 and 9 the round-trip probe's
#else
  LE_TIM(7, 1);
#endif
  LE_TIM(6, (static_cast<uint64_t>(w.b_end - w.b_begin) << 32) | static_cast<uint32_t>(w.part < 0 ? 0 : w.n_parts));
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  // 16-bit tiles: the wave index made provably uniform, so the streaming
  // loop's branches are scalar (fp32 tiles measured faster without it:
  // config 2 20.0 against 20.5 us)
  const int wave = sizeof(KV) == 2 ? __builtin_amdgcn_readfirstlane(tid >> 6) : tid >> 6;
  const int col = lane & 15;   // head of the group (B/C column); key row for A loads
  const int grp = lane >> 4;   // k-group
  const int kvh = by;
  const int G = p.q_heads / p.kv_heads;
  const int bs = p.block_size;
  const int32_t* gtab = p.tables + w.table_off;
  const int kv_stride = p.kv_heads * HD;
  const KV* kc = T::lane_base(p.k_cache, kvh, grp);
  const KV* vc = T::lane_base(p.v_cache, kvh, grp);
  char* vt = lds + wave * T::VT_BYTES;
  // the folded pre-attention RMSNorm: the row's scale, per wave
  float rs = 1.f;
  RowScale<ACT> xs;
  if constexpr (kFold) {
    xs.x = static_cast<const ACT*>(p.rms_x) + static_cast<int64_t>(w.token) * p.rms_hidden;
    xs.hidden = p.rms_hidden;
    xs.eps = p.rms_eps;
    xs.issue();
  } else if (p.rms_x && p.rope_max_pos > 0) {
    rs = row_rms_scale(static_cast<const ACT*>(p.rms_x) + static_cast<int64_t>(w.token) * p.rms_hidden,
                       p.rms_hidden, p.rms_eps);
  }
  store_new_row<KV, kFold>(p, w, kvh, HD, rs, &xs);

  // Q^T (B operand): column `col` = head kvh*G + col.
  typename T::QOp qb;
  {
    const bool ok = col < G;
    const int h = kvh * G + (ok ? col : 0);
    if (kFold || p.rope_max_pos > 0) {
      const bool pos_ok = w.pos >= 0 && w.pos < p.rope_max_pos;  // else q = 0, as rope_kv_write_kernel
      const int64_t tab = static_cast<int64_t>(pos_ok ? w.pos : 0) * (HD / 2);
      const QRope<ACT, kFold> src{
          static_cast<const ACT*>(p.q) + static_cast<int64_t>(w.token) * p.rope_row_stride + h * HD,
          p.rope_bias ? p.rope_bias + h * HD : nullptr, p.rope_cos + tab, p.rope_sin + tab, HD / 2,
          p.rms_x != nullptr, rs, &xs};
      T::load_q(qb, src, ok && pos_ok, grp);
    } else {
      const QRow<ACT> src{static_cast<const ACT*>(p.q) + (static_cast<int64_t>(w.token) * p.q_heads + h) * HD};
      T::load_q(qb, src, ok, grp);
    }
  }

  WaveAcc<HD> st;
#pragma unroll
  for (int d = 0; d < DT; d++) st.acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  st.m = -FLT_MAX;
  st.l = 0.f;

  const int bs_shift = __builtin_ctz(bs);  // block sizes are powers of two
  const int stride = kMfmaWaves * T::kKeys;
  // The partition in segments of at most kTabCap blocks: each segment's
  // block ids are staged in LDS (invalid ids as -1), then streamed. With a
  // plan there is one segment, its ids already in registers and each wave's
  // first tile already in flight.
  for (int sb0 = w.b_begin; sb0 < w.b_end; sb0 += kTabCap) {
    const int sb1 = min(w.b_end, sb0 + kTabCap);
    if (item_ids) {
#pragma unroll
      for (int u = 0; u < kIdsPerThread; u++) {
        const int bid = pre_ids[u];
        tab[tid + u * kMfmaThreads] = (bid >= 0 && bid < p.num_cache_blocks) ? bid : -1;
      }
    } else {
      __syncthreads();  // the previous segment's table is no longer read
      for (int i = tid; i < sb1 - sb0; i += kMfmaThreads) {
        const int bid = gtab[sb0 + i];
        tab[i] = (bid >= 0 && bid < p.num_cache_blocks) ? bid : -1;
      }
    }
    // The workgroup that stores its row's new K/V waits for the store before
    // the barrier, so no wave's later load of that slot precedes it. Only
    // this workgroup reads those lines in the launch: the others do not wait.
    if (stores_new_row(p, w)) __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    LE_TIM(1, LE_TIM_NOW());
    const int key_end = min(sb1 << bs_shift, w.pos + 1);
    int key0 = (sb0 << bs_shift) + wave * T::kKeys;
    if (key0 >= key_end) continue;
    // The early first tile stands unless it holds the key this workgroup
    // stored after issuing it (a partition shorter than the waves' first
    // tiles); the other slots' lines are not touched by the store.
    if (!early || (stores_new_row(p, w) && w.pos < key0 + T::kKeys))
      T::load(ra, kc, vc, key0, key_end, kv_stride, bs_shift, tab, sb0, col);
    if constexpr (kPipe) {
      // The next tile's loads are issued unconditionally (clamped to valid
      // addresses past the end) so every path reaches each compute with the
      // same loads outstanding and the wait before it covers only the tile
      // being computed.
      typename T::Regs rb;
      if constexpr (sizeof(KV) == 2) {
        // This wave's tiles: key0, key0 + stride, ... below key_end (at
        // least one). Pairs run in a loop with one exit and a trip count known
        // at its entry; the last one or two tiles follow it. (A loop with two
        // exits, as below, leaves the compiler's structurizer a dead back
        // edge on which the other buffer's loads are still pending, and the
        // loop head then waits for every load: the two tiles never overlap.
        // 64 x 4096: 27.9 -> 27.3 us.)
        const int n_tiles = (key_end - key0 + stride - 1) / stride;
        const int pairs = (n_tiles - 1) >> 1;
        for (int i = 0; i < pairs; i++) {
          T::load(rb, kc, vc, key0 + stride, key_end, kv_stride, bs_shift, tab, sb0, col);
          T::compute(st, ra, qb, key0, key_end, p.scale_log2, vt, col, grp);
          T::load(ra, kc, vc, key0 + 2 * stride, key_end, kv_stride, bs_shift, tab, sb0, col);
          T::compute(st, rb, qb, key0 + stride, key_end, p.scale_log2, vt, col, grp);
          key0 += 2 * stride;
        }
        T::load(rb, kc, vc, key0 + stride, key_end, kv_stride, bs_shift, tab, sb0, col);
        T::compute(st, ra, qb, key0, key_end, p.scale_log2, vt, col, grp);
        if (n_tiles - 2 * pairs == 2) T::compute(st, rb, qb, key0 + stride, key_end, p.scale_log2, vt, col, grp);
      } else {  // fp32 tiles: the two-exit loop measured faster (config 2 20.0 against 20.5 us)
        while (true) {
          T::load(rb, kc, vc, key0 + stride, key_end, kv_stride, bs_shift, tab, sb0, col);
          T::compute(st, ra, qb, key0, key_end, p.scale_log2, vt, col, grp);
          if (key0 + stride >= key_end) break;
          T::load(ra, kc, vc, key0 + 2 * stride, key_end, kv_stride, bs_shift, tab, sb0, col);
          T::compute(st, rb, qb, key0 + stride, key_end, p.scale_log2, vt, col, grp);
          if (key0 + 2 * stride >= key_end) break;
          key0 += 2 * stride;
        }
      }
    } else {
      while (true) {
        T::compute(st, ra, qb, key0, key_end, p.scale_log2, vt, col, grp);
        key0 += stride;
        if (key0 >= key_end) break;
        T::load(ra, kc, vc, key0, key_end, kv_stride, bs_shift, tab, sb0, col);
      }
    }
  }

  // ---- merge the four waves ----
  LE_TIM(2, LE_TIM_NOW());
#ifndef LE_TIMING_RT
  // every wave's tiles done (slots 8 + wave), in the mixed-step kernel's
  // eight-wave workgroups only: in the decode kernel's unbounded
  // instantiation the extra stores slowed the 64 x 4096 timing build by 19 %
  if constexpr (NW == 8) LE_TIM_WAVE(8, LE_TIM_NOW());
#endif
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
  // Each thread folds the waves' partial results for one 16-byte piece (4
  // dims of a head), with the head's (m, l), and writes the piece straight
  // to the output or the partial: no LDS copy of the folded result and no
  // barrier before the stores.
  for (int c = tid; c < G * HD / 4; c += kMfmaThreads) {
    const int g = c * 4 / HD, d0 = c * 4 - g * HD;
    float M = -FLT_MAX;
#pragma unroll
    for (int v = 0; v < kMfmaWaves; v++) M = fmaxf(M, red[(v * kMaxG + g) * L::RED_STRIDE + HD]);
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    float Ls = 0.f;
#pragma unroll
    for (int v = 0; v < kMfmaWaves; v++) {
      const float* r = red + (v * kMaxG + g) * L::RED_STRIDE;
      const float e = __builtin_amdgcn_exp2f(r[HD] - M);
      o += *reinterpret_cast<const f32x4*>(r + d0) * e;
      Ls += r[HD + 1] * e;
    }
    write_piece<ACT, HD>(p, w, G, kvh, c, o, M, Ls);
  }
  LE_TIM(3, LE_TIM_NOW());
  arrive_and_merge<ACT, HD, kMfmaThreads>(p, w, G, kvh, &sm.flag);
#ifdef LE_TIMING
  __builtin_amdgcn_s_waitcnt(0);  // the merge's output stores are performed
  LE_TIM(4, LE_TIM_NOW());
#endif
}
}  // namespace
}  // namespace dec
}  // namespace le
