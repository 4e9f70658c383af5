// Chunked-prefill attention on MFMA (hot-path part 3, prefill-chunk rows).
//
// Computes the same function as the decode kernel (and the oracle
// ref::paged_attention_head, ops.h:87-111) for the rows of a prefill chunk:
// row t at position pos[t] attends over keys 0..pos[t] of its sequence,
// i.e. causal inside the chunk and over the whole cached prefix before it
// (cpu_model.cpp:144-158 writes every token's K/V before attention runs).
// The reference has no prefill kernel (attention_prefill.cu:1 is a stub) and
// runs chunk rows through the decode kernel, re-reading the history once per
// row; here a tile of 16 consecutive rows shares every K/V read.
//
// gfx950 design:
//   * one 512-thread workgroup (8 waves) per (16-row tile, kv head, key
//     partition); wave w computes query head kv_head*G + w, so one LDS copy
//     of each 64-key K/V tile serves the whole GQA group;
//   * S^T = K . Q^T on v_mfma_f32_16x16x32_bf16: A = K rows from LDS
//     (16 keys x 32 dims per lane-slice), B = Q^T held in registers;
//   * the accumulator layout of S^T puts one query row per lane column, so
//     the online-softmax statistics of a row live in that lane and P^T is
//     already the B operand of the next product, O^T = V^T . P^T, with V
//     transposed into LDS while staging (keys contiguous per dim row);
//   * the k order inside an MFMA is only required to agree between A and B,
//     so P^T's keys {16i + 4g + j} feed the product without any shuffle;
//   * causal mask by absolute position: key kp is live for row t iff
//     kp <= pos[t] and kp is inside the partition; masked scores are -inf,
//     the running max starts at -FLT_MAX, so fully masked tiles add zero.
// bf16 operands, fp32 accumulation; fp32 caches never come here (their chunk
// rows run on the decode kernel for exact fp32 arithmetic).
#include <float.h>

#include "le_common.h"
#include "le_internal.h"

namespace le {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * kWave;
constexpr int kKeys = 64;  // keys per LDS tile

template <int HD> struct ChunkLds {
  static constexpr int K_STRIDE = HD * 2 + 16;    // bytes per key row of K (padded)
  static constexpr int V_STRIDE = kKeys * 2 + 8;  // bytes per dim row of V^T (padded)
  static constexpr int K_BYTES = kKeys * K_STRIDE;
  static constexpr int V_BYTES = HD * V_STRIDE;
};

__device__ __forceinline__ f32x4 mfma16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <typename ACT, int HD>
__global__ __launch_bounds__(kThreads) void chunk_kernel(ChunkParams p) {
  using L = ChunkLds<HD>;
  constexpr int KS = HD / 32;      // MFMA k-steps over head dims
  constexpr int DT = HD / 16;      // 16-dim output tiles
  constexpr int CPR = HD / 8;      // 16-byte chunks per K/V row
  constexpr int LOADS = kKeys * CPR / (kThreads / 2);  // 16-byte loads per staging thread
  static_assert(LOADS >= 1 && kKeys * CPR == LOADS * (kThreads / 2), "staging split");

  __shared__ __attribute__((aligned(16))) char lds_k[L::K_BYTES];
  __shared__ __attribute__((aligned(16))) char lds_v[L::V_BYTES];

  const ChunkItem it = p.items[blockIdx.x];
  const int kvh = blockIdx.y;
  const int G = p.q_heads / p.kv_heads;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid >> 6;
  const int col = lane & 15;  // query row of this lane in the tile
  const int grp = lane >> 4;  // k-group of this lane
  const int bs = p.block_size;
  const bool computes = wave < G;
  const int head = kvh * G + (computes ? wave : 0);
  const int32_t* table = p.tables + p.table_offset[it.seq];
  const int kv_stride = p.kv_heads * HD;

  const bool row_ok = col < it.n_q;
  const int tok = it.tok_begin + (row_ok ? col : 0);
  const int qpos = row_ok ? p.token_pos[tok] : -1;

  // Q^T operand: this lane's 8 dims per k-step of query row `col`, bf16.
  bf16x8 qb[KS];
  {
    const ACT* q = static_cast<const ACT*>(p.q) + (static_cast<int64_t>(tok) * p.q_heads + head) * HD;
#pragma unroll
    for (int ks = 0; ks < KS; ks++)
#pragma unroll
      for (int e = 0; e < 8; e++)
        qb[ks][e] = static_cast<__bf16>(row_ok ? elem<ACT>::load1(q + ks * 32 + grp * 8 + e) : 0.f);
  }

  f32x4 acc[DT];
#pragma unroll
  for (int d = 0; d < DT; d++) acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -FLT_MAX, l_run = 0.f;

  const int key_begin = it.blk_begin * bs;
  const int key_end = it.blk_end * bs;

  // Staging: threads [0, 256) copy K rows, [256, 512) copy V rows (transposed).
  const bool stage_v = tid >= kThreads / 2;
  const int st = tid & (kThreads / 2 - 1);
  const char* kbase = static_cast<const char*>(p.k_cache);
  const char* vbase = static_cast<const char*>(p.v_cache);

  uint4 pre[LOADS];
  auto fetch = [&](int key0) {
#pragma unroll
    for (int i = 0; i < LOADS; i++) {
      const int piece = st + i * (kThreads / 2);
      const int key = piece / CPR, c = piece % CPR;
      const int kp = key0 + key;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (kp < key_end) {
        const int bid = table[kp / bs];
        if (bid >= 0 && bid < p.num_cache_blocks) {
          const int64_t off = ((static_cast<int64_t>(bid) * bs + kp % bs) * kv_stride + kvh * HD + c * 8) * 2;
          v = ld16_stream((stage_v ? vbase : kbase) + off);
        }
      }
      pre[i] = v;
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int i = 0; i < LOADS; i++) {
      const int piece = st + i * (kThreads / 2);
      const int key = piece / CPR, c = piece % CPR;
      if (!stage_v) {
        *reinterpret_cast<uint4*>(lds_k + key * L::K_STRIDE + c * 16) = pre[i];
      } else {
        const uint32_t w[4] = {pre[i].x, pre[i].y, pre[i].z, pre[i].w};
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const uint16_t h = static_cast<uint16_t>(w[e >> 1] >> ((e & 1) * 16));
          *reinterpret_cast<uint16_t*>(lds_v + (c * 8 + e) * L::V_STRIDE + key * 2) = h;
        }
      }
    }
  };

  fetch(key_begin);
  for (int key0 = key_begin; key0 < key_end; key0 += kKeys) {
    __syncthreads();  // the previous tile is no longer read
    stash();
    __syncthreads();
    if (key0 + kKeys < key_end) fetch(key0 + kKeys);  // overlaps with the MFMAs below

    if (computes) {
      // ---- S^T tile: 64 keys x 16 rows, 4 subtiles of 16 keys ----
      f32x4 s[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        s[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(
              lds_k + (i * 16 + col) * L::K_STRIDE + (ks * 32 + grp * 8) * 2);
          s[i] = mfma16x16x32(a, qb[ks], s[i]);
        }
      }
      // scale (log2 domain), mask, tile max of this lane's row
      float mt = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int kp = key0 + i * 16 + grp * 4 + j;
          const bool live = kp <= qpos && kp < key_end;
          const float v = live ? s[i][j] * p.scale_log2 : -INFINITY;
          s[i][j] = v;
          mt = fmaxf(mt, v);
        }
      mt = fmaxf(mt, __shfl_xor(mt, 16, kWave));
      mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
      const float m_new = fmaxf(m_run, mt);
      const float alpha = exp2f(m_run - m_new);
      m_run = m_new;
      float ls = 0.f;
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const float e = exp2f(s[i][j] - m_new);
          s[i][j] = e;
          ls += e;
        }
      l_run = l_run * alpha + ls;  // this lane-group's share; groups merge at the end
#pragma unroll
      for (int d = 0; d < DT; d++) acc[d] *= alpha;

      // ---- O^T += V^T . P^T over the tile's 64 keys (2 k-steps of 32) ----
#pragma unroll
      for (int kk = 0; kk < 2; kk++) {
        bf16x8 pb;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          pb[j] = static_cast<__bf16>(s[2 * kk][j]);
          pb[4 + j] = static_cast<__bf16>(s[2 * kk + 1][j]);
        }
#pragma unroll
        for (int d = 0; d < DT; d++) {
          const char* vr = lds_v + (d * 16 + col) * L::V_STRIDE;
          const bf16x4 lo = *reinterpret_cast<const bf16x4*>(vr + (kk * 32 + grp * 4) * 2);
          const bf16x4 hi = *reinterpret_cast<const bf16x4*>(vr + (kk * 32 + 16 + grp * 4) * 2);
          const bf16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          acc[d] = mfma16x16x32(a, pb, acc[d]);
        }
      }
    }
  }

  if (!computes) return;
  float l_tot = l_run + __shfl_xor(l_run, 16, kWave);
  l_tot += __shfl_xor(l_tot, 32, kWave);
  if (!row_ok) return;

  // acc[d][j] = O[row col][dim d*16 + grp*4 + j]
  if (it.part0 < 0) {
    ACT* out = static_cast<ACT*>(p.out) + (static_cast<int64_t>(tok) * p.q_heads + head) * HD;
    const float inv = 1.f / l_tot;
#pragma unroll
    for (int d = 0; d < DT; d++)
#pragma unroll
      for (int j = 0; j < 4; j++) elem<ACT>::store1(out + d * 16 + grp * 4 + j, acc[d][j] * inv);
  } else {
    const int64_t rec = static_cast<int64_t>(it.part0 + col * it.part_stride) * p.q_heads + head;
    float* dst = p.parts.acc + rec * HD;
#pragma unroll
    for (int d = 0; d < DT; d++)
      *reinterpret_cast<float4*>(dst + d * 16 + grp * 4) =
          make_float4(acc[d][0], acc[d][1], acc[d][2], acc[d][3]);
    if (grp == 0) p.parts.ml[rec] = make_float2(m_run, l_tot);
  }
}

}  // namespace

hipError_t attention_chunk(const ChunkParams& p, int act_bf16, hipStream_t s) {
  if (p.n_items <= 0) return hipSuccess;
  const dim3 grid(p.n_items, p.kv_heads);
  if (p.head_dim == 64) {
    if (act_bf16) chunk_kernel<bf16_t, 64><<<grid, kThreads, 0, s>>>(p);
    else chunk_kernel<float, 64><<<grid, kThreads, 0, s>>>(p);
  } else {
    if (act_bf16) chunk_kernel<bf16_t, 128><<<grid, kThreads, 0, s>>>(p);
    else chunk_kernel<float, 128><<<grid, kThreads, 0, s>>>(p);
  }
  return hipGetLastError();
}

}  // namespace le
