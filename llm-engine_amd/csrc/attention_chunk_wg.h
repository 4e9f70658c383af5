#pragma once
// Chunked-prefill attention on MFMA (hot-path part 3, prefill-chunk rows).
//
// Computes the same function as the decode kernel (and the oracle
// ref::paged_attention_head, ops.h:87-111) for the rows of a prefill chunk:
// row t at position pos[t] attends over keys 0..pos[t] of its sequence,
// i.e. causal inside the chunk and over the whole cached prefix before it
// (cpu_model.cpp:144-158 writes every token's K/V before attention runs).
// The reference has no prefill kernel (attention_prefill.cu:1 is a stub) and
// runs chunk rows through the decode kernel, re-reading the history once per
// row; here 32 consecutive rows share every K/V read.
//
// gfx950 design:
//   * one 512-thread workgroup (8 waves) per (32-row tile, kv head, key
//     partition); wave w computes query head kv_head*G + w for all 32 rows
//     (two 16-row MFMA tiles), so one LDS copy of the keys serves the whole
//     GQA group and both row tiles;
//   * a partition's keys are staged 384 (head_dim 128: 256) at a time: every thread issues its
//     16-byte K and V loads at once (block ids come from the plan, fetched in
//     the same round trip as the item), so a stage costs one memory latency;
//     K and V rows land row-major in LDS;
//   * S^T = K . Q^T on the 16x16x32 MFMA of the cache type, bf16 or fp16 (A = 16 keys x 32 dims from
//     LDS, B = Q^T in registers); the accumulator puts one query row per lane
//     column, so the online-softmax statistics of a row live in that lane and
//     P^T is already the B operand of O^T = V^T . P^T, whose A operand comes
//     from the row-major V tile through the transposing LDS read
//     (ds_read_b64_tr_b16) and is shared by both row tiles;
//   * the k order inside an MFMA is only required to agree between A and B,
//     so P^T's keys {16i + 4g + j} feed the product without any shuffle;
//   * the softmax is the vector-ALU side of a tile (exp2 on every score), so
//     it is kept short: row maxima with v_max3, row sums on the MFMA (a V^T
//     row of ones beside the value tiles), and the running max moves only
//     when a tile's max passes it by more than 8 (log2 units), so the
//     accumulators are rescaled on few tiles and p stays below 2^8
//     (config 3: 25.7 -> 24.9 us per mixed-step launch);
//   * causal mask by absolute position: key kp is live for row t iff
//     kp <= pos[t]; masked scores are -inf and the running max starts at
//     -FLT_MAX, so fully masked tiles add zero;
//   * a tile whose keys were split stores each partition's normalised output
//     (fp16 with a bf16 cache, fp32 otherwise) and its fp32 (max, sum) with
//     device-coherent stores; the last partition to arrive (atomic counter
//     per tile and kv head, reset by it) merges them in partition order,
//     inside the launch.
// 16-bit caches: 16-bit operands (q and P rounded to the cache type), fp32
// accumulation. fp32 caches, head_dim 64: the same tile on the bf16 MFMA with
// every operand in three bf16 terms (products to within the rounding of an
// fp32 product, below), K/V staged 128 keys at a time, the next stage's
// loads in flight during a stage's compute. fp32 caches, head_dim 128: the
// tile on v_mfma_f32_16x16x4_f32 (exact fp32 products), 64 keys a stage.
#include <float.h>

#include <type_traits>

#include "le_common.h"
#include "le_internal.h"

namespace le {
namespace chk {
namespace {


constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kWave;
constexpr int kTileKeys = 64;    // keys per MFMA tile
// fp32 caches with head_dim 64 run on the bf16 MFMA with every operand held
// as three bf16 terms, a = hi + mid + lo (hi = bf16(a), mid = bf16(a - hi),
// lo = bf16(a - hi - mid); both subtractions are exact in fp32), and every
// product as the six terms of order at least 2^-16: hi*hi + hi*mid + mid*hi
// + hi*lo + mid*mid + lo*hi (each exact in the fp32 accumulator). The terms
// left out and lo's rounding are each below 2^-24 |a b|, the size of an fp32
// product's own rounding. The 16x16x32 bf16 MFMA does a product of 32 keys
// or dims at 16 times the fp32 MFMA's rate, so six of them cost 2.7 times
// less than the 16x16x4 fp32 MFMAs they replace. K and V are split once, when
// a stage is stored to LDS, into three bf16 planes; q once per workgroup and
// P per tile in registers. fp32 caches with head_dim 128 keep the fp32 MFMA
// (the three q planes of 128 dims do not fit beside its accumulators).
template <typename KV, int HD> constexpr bool kSplit3 = std::is_same_v<KV, float> && HD == 64;
template <typename KV, int HD> constexpr int kPlanes = kSplit3<KV, HD> ? 3 : 1;
// Keys staged in LDS at once: with a 16-bit cache 384 for head_dim 64 (110 KB
// of K and V rows, so a default 384-key partition is one memory round trip)
// and 256 for head_dim 128 (139 KB); with an fp32 cache 128 for head_dim 64
// (three bf16 planes of K and of V, 110 KB) and 64 for head_dim 128 (68 KB;
// the registers of 128 keys' staging loads do not fit beside the head_dim
// 128 accumulators). Always whole 64-key MFMA tiles.
template <typename KV, int HD>
constexpr int kStageKeys = sizeof(KV) == 2 ? (HD == 64 ? 384 : 256) : (HD == 64 ? 128 : 64);
constexpr int kRowsMax = 32;     // query rows per item
constexpr int kMaxG = 8;         // query heads per kv head
constexpr int kMaxSplit = 16;    // partitions of one tile the merge stages in LDS
constexpr float kRescaleSlack = 8.f;  // log2 units the running max may lag the true max

__device__ __forceinline__ float vmax3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

template <typename KV, int HD> struct ChunkLds {
  // bytes per key row of K and of V (padded); bf16 rows for split fp32
  static constexpr int ROW = HD * (kSplit3<KV, HD> ? 2 : static_cast<int>(sizeof(KV))) + 16;
  static constexpr int PLANE = kStageKeys<KV, HD> * ROW;  // one plane of the stage's K or V rows
  static constexpr int K_BYTES = kPlanes<KV, HD> * PLANE;
  static constexpr int BYTES = 2 * K_BYTES;  // K rows (planes hi, mid, lo), then V rows
};

// a = hi + mid + lo in bf16 terms (the split of the fp32 path above)
struct Bf3 { __bf16 hi, mid, lo; };
__device__ __forceinline__ Bf3 split3(float a) {
  Bf3 t;
  t.hi = static_cast<__bf16>(a);
  const float r = a - static_cast<float>(t.hi);
  t.mid = static_cast<__bf16>(r);
  t.lo = static_cast<__bf16>(r - static_cast<float>(t.mid));
  return t;
}
// element e of three operand vectors from one split
template <typename V>
__device__ __forceinline__ void put3(V& h, V& m, V& l, int e, float a) {
  const Bf3 t = split3(a);
  h[e] = t.hi;
  m[e] = t.mid;
  l[e] = t.lo;
}

__device__ __forceinline__ void st_dev(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_dev(const float* p) {
  return __uint_as_float(__hip_atomic_load(reinterpret_cast<uint32_t*>(const_cast<float*>(p)),
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}


template <typename ACT>
__device__ __forceinline__ void store4(ACT* p, f32x4 v) {
  const float f[4] = {v[0], v[1], v[2], v[3]};
  elem<ACT>::store4(p, f);
}

// LDS of one chunk workgroup.
template <typename KV, int HD> struct ChunkSmem {
  __attribute__((aligned(16))) char lds[ChunkLds<KV, HD>::BYTES];
  int last;
};

// The last partition's merge of a split tile. Each thread owns kMG output
// 8-vectors (a row, a head, 8 consecutive dims) and merges their partials
// itself, kMJ partitions per round of loads: the partition's (m, l) for the
// row and head, and its normalised output (fp32), requested together, then
// folded in partition order into a running (max, sum) with rescaling. With at
// most kMJ partitions the whole merge is one memory round trip, with no LDS
// phase or barrier.
// Split tiles of a bf16 cache carry their partials as fp16: the tile already
// rounds its softmax weights to bf16 (2^-9), and a normalised partial is a
// convex combination of V rows, so rounding it to fp16 moves the merged output
// by at most 2^-11 max|V|; it halves the partial store and the merge's loads.
// The price is the fp16 range, the reference's own cache range: a partial
// element past 65504 (only possible with |V| > 65504 in the cache) becomes
// inf, so the row's output comes back inf or NaN, never a wrong finite value.
// fp16 and fp32 caches keep fp32 partials.
template <typename KV> constexpr bool kHalfPartials = std::is_same_v<KV, bf16_t>;

template <typename ACT, int HD, int kMJ, bool kHalf>
__device__ __forceinline__ void merge_tile(const ChunkParams& p, const ChunkItem& it, __amdgpu_buffer_rsrc_t acc_rsrc,
                                           float* ml, int64_t rec_tile, int base, int J, int G, int kvh, int nq,
                                           int tok0) {
  constexpr int kMG = 2;  // output 8-vectors per thread and round
  const int tid = threadIdx.x;
  const int per_row = G * (HD / 8);
  const int n_out = nq * per_row;
  for (int o0 = tid; o0 < n_out; o0 += kMG * kThreads) {
    int64_t rec_base[kMG];
    int d8[kMG];
    float M[kMG], L[kMG], sum[kMG][8];
#pragma unroll
    for (int gi = 0; gi < kMG; gi++) {
      const int o = min(o0 + gi * kThreads, n_out - 1);
      const int r = o / per_row, rem = o - r * per_row;
      const int g = rem / (HD / 8);
      d8[gi] = rem - g * (HD / 8);
      rec_base[gi] = static_cast<int64_t>(base + r * J) * p.q_heads + kvh * G + g;
      M[gi] = -FLT_MAX;
      L[gi] = 0.f;
#pragma unroll
      for (int e = 0; e < 8; e++) sum[gi][e] = 0.f;
    }
    for (int j0 = 0; j0 < J; j0 += kMJ) {
      f32x4 x[kMG][kMJ][2];
      uint4 xh[kMG][kMJ];
      float mj[kMG][kMJ], lj[kMG][kMJ];
#pragma unroll
      for (int gi = 0; gi < kMG; gi++)
#pragma unroll
        for (int jj = 0; jj < kMJ; jj++) {
          const int64_t rec = rec_base[gi] + static_cast<int64_t>(min(j0 + jj, J - 1)) * p.q_heads;
          if constexpr (kHalf) {
            xh[gi][jj] = ld_coherent16u(acc_rsrc, static_cast<uint32_t>(((rec - rec_tile) * HD + d8[gi] * 8) * 2));
          } else {
            const uint32_t off = static_cast<uint32_t>(((rec - rec_tile) * HD + d8[gi] * 8) * 4);
            x[gi][jj][0] = ld_coherent16(acc_rsrc, off);
            x[gi][jj][1] = ld_coherent16(acc_rsrc, off + 16);
          }
          mj[gi][jj] = ld_dev(ml + rec * 2);
          lj[gi][jj] = ld_dev(ml + rec * 2 + 1);
        }
      if constexpr (kHalf) {
#pragma unroll
        for (int gi = 0; gi < kMG; gi++)
#pragma unroll
          for (int jj = 0; jj < kMJ; jj++) {
            float f[8];
            elem<f16_t>::widen(xh[gi][jj], f);
            x[gi][jj][0] = f32x4{f[0], f[1], f[2], f[3]};
            x[gi][jj][1] = f32x4{f[4], f[5], f[6], f[7]};
          }
      }
#pragma unroll
      for (int gi = 0; gi < kMG; gi++)
#pragma unroll
        for (int jj = 0; jj < kMJ; jj++)
          if (j0 + jj < J) {
            // partition j holds o_j / l_j; fold in l_j * o_j at weight exp2(m_j - max)
            const float m_new = fmaxf(M[gi], mj[gi][jj]);
            const float a = __builtin_amdgcn_exp2f(M[gi] - m_new), w = __builtin_amdgcn_exp2f(mj[gi][jj] - m_new) * lj[gi][jj];
            M[gi] = m_new;
            L[gi] = L[gi] * a + w;
#pragma unroll
            for (int e = 0; e < 8; e++) sum[gi][e] = sum[gi][e] * a + w * x[gi][jj][e >> 2][e & 3];
          }
    }
#pragma unroll
    for (int gi = 0; gi < kMG; gi++) {
      const int o = o0 + gi * kThreads;
      if (o < n_out) {
        const int r = o / per_row, rem = o - r * per_row;
        const int g = rem / (HD / 8);
        ACT* out = static_cast<ACT*>(p.out) + (static_cast<int64_t>(tok0 + r) * p.q_heads + kvh * G + g) * HD + d8[gi] * 8;
        const float inv = 1.f / L[gi];
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = sum[gi][e] * inv;
        elem<ACT>::store8(out, v);
      }
    }
  }
}

// One chunk workgroup (kThreads threads): chunk item `item`, kv head `kvh`.
// Shared by the chunk kernel and the fused ragged kernel.
template <typename ACT, typename KV, int HD>
__device__ __forceinline__ void chunk_wg(const ChunkParams& p, ChunkSmem<KV, HD>& sm, int item, int kvh) {
  // 16-bit caches: the 16x16x32 MFMA of the cache type (q and P rounded to
  // it). fp32 caches: the bf16 MFMA on three-term operands (head_dim 64) or
  // v_mfma_f32_16x16x4_f32, exact fp32 products (head_dim 128).
  constexpr bool kSplit = kSplit3<KV, HD>;                    // fp32 operands as three bf16 terms
  constexpr bool kF32 = std::is_same_v<KV, float> && !kSplit;  // fp32 operands on the fp32 MFMA
  using M = mma16<std::conditional_t<std::is_same_v<KV, float>, bf16_t, KV>>;
  using V8 = typename M::v8;
  using S16 = typename M::scalar;
  using L = ChunkLds<KV, HD>;
  constexpr int KS = HD / 32;  // 16-bit MFMA k-steps over head dims
  constexpr int DT = HD / 16;  // 16-dim output tiles
  constexpr int LD = HD / 4;   // fp32: dims per lane group (contiguous), one per MFMA k-step
  constexpr int CPR = HD * static_cast<int>(sizeof(KV)) / 16;  // 16-byte pieces per K/V row
  constexpr int PIECES = 2 * kStageKeys<KV, HD> * CPR;
  constexpr int PER = PIECES / kThreads;  // 16-byte loads per thread per stage
  static_assert(PER * kThreads == PIECES && PER % 2 == 0, "staging split");
  static_assert(kStageKeys<KV, HD> % kTileKeys == 0, "a stage is whole MFMA tiles");
  static_assert(kRowsMax * kMaxG * kMaxSplit * (sizeof(float2) + sizeof(float)) <= L::BYTES,
                "merge weights fit in the stage's LDS");

  char* lds = sm.lds;
  int& last = sm.last;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int col = lane & 15;  // query row of this lane within a 16-row tile
  const int grp = lane >> 4;  // k-group of this lane
  [[maybe_unused]] const uint64_t t_start = LE_TIM_NOW();
  const ChunkItem it = p.items[item];
  if (it.n_q <= 0) return;  // padding that keeps split tiles on one XCD
  LE_TIM(0, t_start);
  LE_TIM(5, LE_TIM_PLACE());
  LE_TIM(6, (static_cast<uint64_t>(it.blk_end - it.blk_begin) << 32) | static_cast<uint32_t>(it.part0 < 0 ? 0 : it.part_stride));
  LE_TIM(7, 2);
  const int G = p.q_heads / p.kv_heads;
  const bool computes = wave < G;
  const int head = kvh * G + (computes ? wave : 0);
  const int bs_shift = __builtin_ctz(p.block_size);  // block sizes are powers of two
  const int bs_mask = p.block_size - 1;
  const int nq = it.n_q;
  const int tok0 = it.tok_begin;
  const int kv_stride = p.kv_heads * HD;
  const int key_begin = it.blk_begin << bs_shift;
  // The item's block ids sit at a fixed stride in the plan, padded with -1:
  // each thread reads the ids of its own keys there directly, so the K/V
  // loads wait for one round trip and no barrier.
  const int32_t* ids = p.item_ids + static_cast<int64_t>(item) * p.ids_stride;
  const char* kbase = static_cast<const char*>(p.k_cache);
  const char* vbase = static_cast<const char*>(p.v_cache);

  // Stage staging: thread pieces k cover key (tid + k*kThreads) / CPR, 16-byte
  // piece c of that key's K row and of its V row. Keys past the item's live
  // keys (the unused rows of its last block, which may hold anything, NaN
  // included) or in an invalid block read the item's last live key instead
  // and are stored as zeros: their scores are masked, and a zero V row keeps
  // p * v finite.
  uint4 kv[2][PER / 2];
  bool okp[PER / 2];
  auto issue = [&](int rel0) {
#pragma unroll
    for (int k = 0; k < PER / 2; k++) {
      const int piece = tid + k * kThreads;
      const int key_l = piece / CPR, c = piece - key_l * CPR;
      // a piece past the item reads the item's last live key instead (a line
      // the workgroup loads anyway), not one shared address that every
      // workgroup's surplus pieces would pile onto
      const int rel = rel0 + key_l;
      const int relc = min(rel, it.key_live - 1);
      const int bid = ids[min(relc >> bs_shift, p.ids_stride - 1)];
      const bool bid_ok = bid >= 0 && bid < p.num_cache_blocks;
      okp[k] = rel < it.key_live && bid_ok;
      const int64_t slot = (static_cast<int64_t>(bid_ok ? bid : 0) << bs_shift) + (relc & bs_mask);
      const int64_t off = (slot * kv_stride + kvh * HD) * static_cast<int64_t>(sizeof(KV)) + c * 16;
      kv[0][k] = ld16_stream(kbase + off);
      kv[1][k] = ld16_stream(vbase + off);
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int k = 0; k < PER / 2; k++) {
      const int piece = tid + k * kThreads;  // as in issue(): the LDS place is recomputed, not kept
      const int key_l = piece / CPR, c = piece - key_l * CPR;
      if constexpr (kSplit) {
        // four fp32 dims become 8 bytes in each of the three bf16 planes
        const int dst = key_l * L::ROW + c * 8;
#pragma unroll
        for (int kv_i = 0; kv_i < 2; kv_i++) {
          const uint4 u = okp[k] ? kv[kv_i][k] : make_uint4(0, 0, 0, 0);
          const float f[4] = {__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w)};
          typename M::v4 h, m, l;
#pragma unroll
          for (int e = 0; e < 4; e++) put3(h, m, l, e, f[e]);
          char* base = lds + kv_i * L::K_BYTES + dst;
          *reinterpret_cast<typename M::v4*>(base) = h;
          *reinterpret_cast<typename M::v4*>(base + L::PLANE) = m;
          *reinterpret_cast<typename M::v4*>(base + 2 * L::PLANE) = l;
        }
      } else {
        const int dst = key_l * L::ROW + c * 16;
        *reinterpret_cast<uint4*>(lds + dst) = okp[k] ? kv[0][k] : make_uint4(0, 0, 0, 0);
        *reinterpret_cast<uint4*>(lds + L::K_BYTES + dst) = okp[k] ? kv[1][k] : make_uint4(0, 0, 0, 0);
      }
    }
  };
  // Query rows first (they are needed last, and a wait for them must not
  // cover the K/V loads issued after them), then the stage's K/V.
  const int pos0 = p.token_pos[tok0];  // the tile's rows are consecutive positions
  // 16-bit path: this lane's 8 dims per k-step (dims ks*32 + grp*8 ..);
  // fp32 path: this lane's LD contiguous dims (grp*LD ..). Loaded raw before
  // the stage's K/V loads are issued, converted after.
  constexpr int QPIECES = (kF32 ? LD : KS * 8) / 8;  // 8-element pieces per row and lane
  float qf[2][QPIECES * 8];
  uint4 qraw[2][QPIECES][sizeof(ACT) / 2];
#pragma unroll
  for (int rs = 0; rs < 2; rs++) {
    const int r = rs * 16 + col;
    const bool ok = computes && r < nq;
    const ACT* q = static_cast<const ACT*>(p.q) + (static_cast<int64_t>(tok0 + (ok ? r : 0)) * p.q_heads + head) * HD;
#pragma unroll
    for (int u = 0; u < QPIECES; u++) {
      const int d0 = kF32 ? grp * LD + u * 8 : u * 32 + grp * 8;
#pragma unroll
      for (int h = 0; h < static_cast<int>(sizeof(ACT) / 2); h++) qraw[rs][u][h] = ld16(q + d0 + h * (16 / sizeof(ACT)));
    }
  }
  issue(0);
#pragma unroll
  for (int rs = 0; rs < 2; rs++) {
    const bool ok = computes && rs * 16 + col < nq;
#pragma unroll
    for (int u = 0; u < QPIECES; u++) {
      float f[8];
      if constexpr (sizeof(ACT) == 2) {
        elem<ACT>::widen(qraw[rs][u][0], f);
      } else {
        elem<float>::widen(qraw[rs][u][0], f);
        elem<float>::widen(qraw[rs][u][1], f + 4);
      }
#pragma unroll
      for (int e = 0; e < 8; e++) qf[rs][u * 8 + e] = ok ? f[e] * p.scale_log2 : 0.f;
    }
  }
  // 16-bit path: Q^T operands, this lane's 8 dims per k-step of rows col and
  // 16 + col (split fp32: qb, qm, ql the three terms)
  V8 qb[2][KS];
  [[maybe_unused]] V8 qm[2][KS], ql[2][KS];
  if constexpr (!kF32) {
#pragma unroll
    for (int rs = 0; rs < 2; rs++)
#pragma unroll
      for (int ks = 0; ks < KS; ks++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
          if constexpr (kSplit) put3(qb[rs][ks], qm[rs][ks], ql[rs][ks], e, qf[rs][ks * 8 + e]);
          else qb[rs][ks][e] = static_cast<S16>(qf[rs][ks * 8 + e]);
        }
  }

  f32x4 acc[2][DT];
#pragma unroll
  for (int rs = 0; rs < 2; rs++)
#pragma unroll
    for (int d = 0; d < DT; d++) acc[rs][d] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[2] = {-FLT_MAX, -FLT_MAX};
  // The S^T accumulators start at -sbase (per row): scores come out of the
  // MFMA as s - sbase, already in log2 units (q carries scale * log2(e)).
  // sbase is the running max once the row has a live key (0 before), so on
  // tiles that do not move the max, p = exp2(s - sbase) with no vector-ALU
  // work before the exp2.
  float sbase[2] = {0.f, 0.f};
  f32x4 nbase[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};  // -sbase, the MFMA's C operand
  // 16-bit path: lsum[rs][0] of the lanes of group 0 = the row's sum of p
  // (row col), summed on the MFMA; the other entries stay zero. fp32 paths:
  // lsum[rs][0] of every lane = its share of the row's sum (the keys of its
  // lane group). Either way the row sum is lsum[rs][0] summed over the four
  // lane groups.
  f32x4 lsum[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  const S16 one = static_cast<S16>(col == 0 ? 1.f : 0.f);
  const V8 ones = {one, one, one, one, one, one, one, one};

  for (int rel0 = 0;;) {
    stash();
    __syncthreads();
    if (rel0 == 0) LE_TIM(1, LE_TIM_NOW());
    // split fp32: the next stage's loads leave before this stage's compute
    if constexpr (kSplit)
      if (rel0 + kStageKeys<KV, HD> < it.key_live) issue(rel0 + kStageKeys<KV, HD>);
    const int s0 = key_begin + rel0;
    if (computes) {
      const int key_end = key_begin + it.key_live;  // past the last row's position: dead
      // Tiles of the stage with a live key.
      const int nt = min(kStageKeys<KV, HD> / kTileKeys, (key_end - s0 + kTileKeys - 1) / kTileKeys);
      // ---- S^T of tile kt: 64 keys x 32 rows, less the rows' current base ----
      auto scores = [&](int kt, f32x4 (&s)[2][4]) {
        const char* kt_lds = lds + kt * kTileKeys * L::ROW;
#pragma unroll
        for (int rs = 0; rs < 2; rs++)
#pragma unroll
          for (int i = 0; i < 4; i++) s[rs][i] = nbase[rs];
        if constexpr (kSplit) {
          // per 16 keys x 32 dims: the three K terms, then both row tiles'
          // six products, smallest terms first
#pragma unroll
          for (int i = 0; i < 4; i++)
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
              const char* kp = kt_lds + (i * 16 + col) * L::ROW + (ks * 32 + grp * 8) * 2;
              const V8 kh = *reinterpret_cast<const V8*>(kp);
              const V8 km = *reinterpret_cast<const V8*>(kp + L::PLANE);
              const V8 kl = *reinterpret_cast<const V8*>(kp + 2 * L::PLANE);
#pragma unroll
              for (int rs = 0; rs < 2; rs++) {
                s[rs][i] = M::mma(kl, qb[rs][ks], s[rs][i]);
                s[rs][i] = M::mma(km, qm[rs][ks], s[rs][i]);
                s[rs][i] = M::mma(kh, ql[rs][ks], s[rs][i]);
                s[rs][i] = M::mma(km, qb[rs][ks], s[rs][i]);
                s[rs][i] = M::mma(kh, qm[rs][ks], s[rs][i]);
                s[rs][i] = M::mma(kh, qb[rs][ks], s[rs][i]);
              }
            }
        } else if constexpr (!kF32) {
          // the tile's K fragments, then row tile 0's products before row
          // tile 1's: the softmax of row tile 0 starts while row tile 1's
          // products are still in the MFMA pipe
          V8 ka[4][KS];
#pragma unroll
          for (int i = 0; i < 4; i++)
#pragma unroll
            for (int ks = 0; ks < KS; ks++)
              ka[i][ks] = *reinterpret_cast<const V8*>(kt_lds + (i * 16 + col) * L::ROW + (ks * 32 + grp * 8) * 2);
#pragma unroll
          for (int rs = 0; rs < 2; rs++)
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
              for (int ks = 0; ks < KS; ks++) s[rs][i] = M::mma(ka[i][ks], qb[rs][ks], s[rs][i]);
        } else {
          // k-step j: dim grp*LD + j of key col (A) and of row col (B); the
          // steps and lane groups together cover every dim once
#pragma unroll
          for (int i = 0; i < 4; i++) {
            float kf[LD];
#pragma unroll
            for (int u = 0; u < LD / 4; u++) {
              const float4 v = *reinterpret_cast<const float4*>(kt_lds + (i * 16 + col) * L::ROW + (grp * LD + u * 4) * 4);
              kf[u * 4] = v.x; kf[u * 4 + 1] = v.y; kf[u * 4 + 2] = v.z; kf[u * 4 + 3] = v.w;
            }
#pragma unroll
            for (int j = 0; j < LD; j++)
#pragma unroll
              for (int rs = 0; rs < 2; rs++)
                s[rs][i] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[j], qf[rs][j], s[rs][i], 0, 0, 0);
          }
        }
      };
      auto soft_pv = [&](int kt, f32x4 (&s)[2][4]) {
        const int t0 = s0 + kt * kTileKeys;
        const char* vt_lds = lds + L::K_BYTES + kt * kTileKeys * L::ROW;
        // ---- causal mask, online softmax per row (log2 domain) ----
        // A tile wholly below the diagonal and inside the range needs no
        // mask: every row's position is at least pos0. Arguments of exp2 are
        // at most kRescaleSlack, so the raw hardware exp2 (whose results
        // below 2^-126 flush to zero) suffices.
        const bool full = t0 + kTileKeys - 1 <= pos0 && t0 + kTileKeys <= key_end;
        auto softmax = [&](int rs) {
          if (!full) {
            // key t0 + 16i + 4grp + j is live iff 16i + j <= lim: one
            // per-lane limit against compile-time offsets
            const int r = rs * 16 + col;
            const int qpos = r < nq ? pos0 + r : -1;
            const int lim = min(qpos, key_end - 1) - t0 - grp * 4;
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
              for (int j = 0; j < 4; j++)
                if (i * 16 + j > lim) s[rs][i][j] = -INFINITY;
          }
          // a tree of v_max3 (depth 3) over the lane's 16 scores
          const float m0 = vmax3(s[rs][0][0], s[rs][0][1], s[rs][0][2]);
          const float m1 = vmax3(s[rs][0][3], s[rs][1][0], s[rs][1][1]);
          const float m2 = vmax3(s[rs][1][2], s[rs][1][3], s[rs][2][0]);
          const float m3 = vmax3(s[rs][2][1], s[rs][2][2], s[rs][2][3]);
          const float m4 = vmax3(s[rs][3][0], s[rs][3][1], s[rs][3][2]);
          float mt = vmax2(vmax3(m0, m1, m2), vmax3(m3, m4, s[rs][3][3]));
          // The running max moves only when the tile's max passes it by more
          // than kRescaleSlack (log2 units): probabilities then stay below
          // 2^kRescaleSlack, and the accumulators are rescaled and the
          // scores shifted to the new base only on the tiles where some row
          // of the wave moved its max (always on a row's first live tile).
          // A row that does not move keeps sbase == m_run, or has only
          // masked (-inf) scores so far. The test runs on each lane's own
          // 16 scores; only when some lane passes it is the row's maximum
          // over its four lanes formed.
          if (__builtin_amdgcn_ballot_w64(mt + sbase[rs] > m_run[rs] + kRescaleSlack)) {
            const float cand = rows_max(mt) + sbase[rs];
            const bool grow = cand > m_run[rs] + kRescaleSlack;
            const float m_new = grow ? cand : m_run[rs];
            const float alpha = __builtin_amdgcn_exp2f(m_run[rs] - m_new);
            const float shift = grow ? m_new - sbase[rs] : 0.f;
            m_run[rs] = m_new;
            sbase[rs] = grow ? m_new : sbase[rs];
            nbase[rs] = f32x4{-sbase[rs], -sbase[rs], -sbase[rs], -sbase[rs]};
#pragma unroll
            for (int d = 0; d < DT; d++) acc[rs][d] *= alpha;
            lsum[rs] *= alpha;
#pragma unroll
            for (int i = 0; i < 4; i++) s[rs][i] -= shift;
          }
#pragma unroll
          for (int i = 0; i < 4; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) s[rs][i][j] = __builtin_amdgcn_exp2f(s[rs][i][j]);
        };
        if constexpr (kSplit) {
          softmax(0);
          softmax(1);
          // ---- O^T += V^T . P^T as in the 16-bit path, each operand in three
          // bf16 terms (P^T split here, V^T read from the three planes) ----
#pragma unroll
          for (int kk = 0; kk < 2; kk++) {
            V8 ph[2], pm[2], pl[2];
#pragma unroll
            for (int rs = 0; rs < 2; rs++)
#pragma unroll
              for (int j = 0; j < 4; j++) {
                put3(ph[rs], pm[rs], pl[rs], j, s[rs][2 * kk][j]);
                put3(ph[rs], pm[rs], pl[rs], 4 + j, s[rs][2 * kk + 1][j]);
              }
            const char* r_lo = vt_lds + (kk * 32 + grp * 4 + (col >> 2)) * L::ROW + (col & 3) * 8;
            const char* r_hi = r_lo + 16 * L::ROW;
#pragma unroll
            for (int d = 0; d < DT; d++) {
              V8 v3[3];
#pragma unroll
              for (int pl_i = 0; pl_i < 3; pl_i++) {
                const typename M::v4 lo = lds_read_tr16<bf16_t>(r_lo + pl_i * L::PLANE + d * 32);
                const typename M::v4 hi = lds_read_tr16<bf16_t>(r_hi + pl_i * L::PLANE + d * 32);
                v3[pl_i] = V8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
              }
#pragma unroll
              for (int rs = 0; rs < 2; rs++) {
                acc[rs][d] = M::mma(v3[2], ph[rs], acc[rs][d]);
                acc[rs][d] = M::mma(v3[1], pm[rs], acc[rs][d]);
                acc[rs][d] = M::mma(v3[0], pl[rs], acc[rs][d]);
                acc[rs][d] = M::mma(v3[1], ph[rs], acc[rs][d]);
                acc[rs][d] = M::mma(v3[0], pm[rs], acc[rs][d]);
                acc[rs][d] = M::mma(v3[0], ph[rs], acc[rs][d]);
              }
            }
          }
          // row sums of the fp32 p, per lane group as in the fp32 path
#pragma unroll
          for (int rs = 0; rs < 2; rs++) {
            float ls = 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++) ls += (s[rs][i][0] + s[rs][i][1]) + (s[rs][i][2] + s[rs][i][3]);
            lsum[rs][0] += ls;
          }
        } else if constexpr (!kF32) {
          // ---- O^T += V^T . P^T over the tile's 64 keys (2 k-steps of 32) ----
          // V^T operands for both row tiles, read once: lane (col, grp)
          // addresses key row kk*32 + 4*grp + col/4 (then +16) at dims
          // 16*d + 4*(col%4), and receives dim 16*d + col of four keys: the
          // keys P^T holds for that group.
          V8 va[2][DT];
#pragma unroll
          for (int kk = 0; kk < 2; kk++) {
            const char* r_lo = vt_lds + (kk * 32 + grp * 4 + (col >> 2)) * L::ROW + (col & 3) * 8;
            const char* r_hi = r_lo + 16 * L::ROW;
#pragma unroll
            for (int d = 0; d < DT; d++) {
              const typename M::v4 lo = lds_read_tr16<KV>(r_lo + d * 32);
              const typename M::v4 hi = lds_read_tr16<KV>(r_hi + d * 32);
              va[kk][d] = V8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
          }
          auto pv = [&](int rs) {
#pragma unroll
            for (int kk = 0; kk < 2; kk++) {
              V8 pb;
#pragma unroll
              for (int j = 0; j < 4; j++) {
                pb[j] = static_cast<S16>(s[rs][2 * kk][j]);
                pb[4 + j] = static_cast<S16>(s[rs][2 * kk + 1][j]);
              }
#pragma unroll
              for (int d = 0; d < DT; d++) acc[rs][d] = M::mma(va[kk][d], pb, acc[rs][d]);
              // row sums on the MFMA: a V^T row of ones (lanes of column 0)
              lsum[rs] = M::mma(ones, pb, lsum[rs]);
            }
          };
          // row tile 1's softmax runs while row tile 0's products are in
          // the MFMA pipe
          softmax(0);
          pv(0);
          softmax(1);
          pv(1);
        } else {
          softmax(0);
          softmax(1);
          // ---- O^T += V^T . P^T: k-step (i, r) covers keys 16i + 4*grp + r,
          // exactly the scores this lane's S^T accumulators hold, so P^T is
          // the accumulator as is; V^T reads single floats of the row-major
          // V rows (the 16-byte row pad spreads the lane groups' rows over
          // the banks) ----
#pragma unroll
          for (int i = 0; i < 4; i++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
              const float* vrow = reinterpret_cast<const float*>(vt_lds + (i * 16 + grp * 4 + r) * L::ROW);
#pragma unroll
              for (int d = 0; d < DT; d++) {
                const float a = vrow[d * 16 + col];
#pragma unroll
                for (int rs = 0; rs < 2; rs++)
                  acc[rs][d] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, s[rs][i][r], acc[rs][d], 0, 0, 0);
              }
            }
#pragma unroll
          for (int rs = 0; rs < 2; rs++) {
            float ls = 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++) ls += (s[rs][i][0] + s[rs][i][1]) + (s[rs][i][2] + s[rs][i][3]);
            lsum[rs][0] += ls;
          }
        }
      };
#pragma unroll 1
      for (int kt = 0; kt < nt; kt++) {
        f32x4 sa[2][4];
        scores(kt, sa);
        soft_pv(kt, sa);
      }
    }
    rel0 += kStageKeys<KV, HD>;
    if (rel0 >= it.key_live) break;
    __syncthreads();  // the stage is no longer read
    if constexpr (!kSplit) issue(rel0);
  }

  LE_TIM(2, LE_TIM_NOW());
  LE_TIM_WAVE(8, LE_TIM_NOW());
  // acc[rs][d][j] = O[row rs*16 + col][dim d*16 + grp*4 + j]
  float l_tot[2];
#pragma unroll
  for (int rs = 0; rs < 2; rs++) {
    l_tot[rs] = rows_sum(lsum[rs][0]);
  }
  if (it.part0 < 0) {
    if (computes) {
#pragma unroll
      for (int rs = 0; rs < 2; rs++) {
        const int r = rs * 16 + col;
        if (r < nq) {
          ACT* out = static_cast<ACT*>(p.out) + (static_cast<int64_t>(tok0 + r) * p.q_heads + head) * HD;
          const float inv = 1.f / l_tot[rs];
#pragma unroll
          for (int d = 0; d < DT; d++) store4<ACT>(out + d * 16 + grp * 4, acc[rs][d] * inv);
        }
      }
    }
#ifdef LE_TIMING
    __builtin_amdgcn_s_waitcnt(0);
    LE_TIM(3, LE_TIM_NOW());
    LE_TIM(4, LE_TIM_NOW());
#endif
    return;
  }

  // ---- split tile: store the partial, then the last partition merges ----
  // The tile's partial records start at record (part0 - part) * q_heads:
  // offsets from there stay far below the buffer descriptor's 2 GB range
  // however large the workspace is.
  const int64_t rec_tile = static_cast<int64_t>(it.part0 - it.part) * p.q_heads;
  const __amdgpu_buffer_rsrc_t acc_rsrc = coherent_rsrc(p.parts.acc + rec_tile * HD);
  float* ml = reinterpret_cast<float*>(p.parts.ml);
  if (computes) {
#pragma unroll
    for (int rs = 0; rs < 2; rs++) {
      const int r = rs * 16 + col;
      if (r < nq) {
        const int64_t rec = static_cast<int64_t>(it.part0 + r * it.part_stride) * p.q_heads + head;
        // the partition's normalised output (fp16 or fp32), in the record's natural
        // layout (a row with no live key in the partition stores zeros and
        // l = 0): lane (col, grp) holds dims d*16 + grp*4 .. +4 of each
        // output tile d
        const float inv = l_tot[rs] > 0.f ? 1.f / l_tot[rs] : 0.f;
#pragma unroll
        for (int d = 0; d < DT; d++) {
          const f32x4 o = acc[rs][d] * inv;
          if constexpr (kHalfPartials<KV>) {
            const uint32_t off = static_cast<uint32_t>(((rec - rec_tile) * HD + d * 16 + grp * 4) * 2);
            const uint2 v = make_uint2(pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3]));
            if (p.l2_local) st_l2_8(acc_rsrc, off, v);
            else st_coherent8(acc_rsrc, off, v);
          } else {
            const uint32_t off = static_cast<uint32_t>(((rec - rec_tile) * HD + d * 16 + grp * 4) * 4);
            const f32x4v v = __builtin_bit_cast(f32x4v, o);
            if (p.l2_local) st_l2_16(acc_rsrc, off, v);
            else st_coherent16(acc_rsrc, off, v);
          }
        }
        if (grp == 0) {
          if (p.l2_local) {  // the tile's partitions share this XCD's L2
            reinterpret_cast<float2*>(ml)[rec] = make_float2(m_run[rs], l_tot[rs]);
          } else {
            st_dev(ml + rec * 2, m_run[rs]);
            st_dev(ml + rec * 2 + 1, l_tot[rs]);
          }
        }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores are performed
  __syncthreads();                // ... and every other thread's
  LE_TIM(3, LE_TIM_NOW());
  arrival_t* counter = p.parts.counters + static_cast<int64_t>(tok0) * p.kv_heads + kvh;
  if (tid == 0) {
    const arrival_t seen = __hip_atomic_fetch_add(counter, arrival_t{1}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = seen == static_cast<arrival_t>(it.part_stride - 1);
  }
  __syncthreads();
#ifdef LE_TIMING
  if (!last) LE_TIM(4, LE_TIM_NOW());
#endif
  if (!last) return;

  // Every other partition incremented the counter after its partials were
  // performed, so the coherent loads of the merge see all of them.
  const int J = it.part_stride;
  const int base = it.part0 - it.part;
  // Rounds of loads as wide as the tile's partition count (up to 6 for hd
  // 64), so no load is issued twice.
  if constexpr (HD == 64) {
    if (J <= 4) merge_tile<ACT, HD, 4, kHalfPartials<KV>>(p, it, acc_rsrc, ml, rec_tile, base, J, G, kvh, nq, tok0);
    else merge_tile<ACT, HD, 6, kHalfPartials<KV>>(p, it, acc_rsrc, ml, rec_tile, base, J, G, kvh, nq, tok0);
  } else {
    merge_tile<ACT, HD, 3, kHalfPartials<KV>>(p, it, acc_rsrc, ml, rec_tile, base, J, G, kvh, nq, tok0);
  }
  if (tid == 0) __hip_atomic_store(counter, arrival_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#ifdef LE_TIMING
  __builtin_amdgcn_s_waitcnt(0);  // the merge's output stores are performed
  LE_TIM(4, LE_TIM_NOW());
#endif
}
}  // namespace
}  // namespace chk
}  // namespace le
