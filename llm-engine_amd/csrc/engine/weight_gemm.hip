// Weight-streaming GEMM for decode steps: Y[m][n] = X[m][k] . W[n][k]^T with
// few rows (m <= 64 tokens), bf16 operands, fp32 accumulation.
//
// The reference multiplies through cuBLAS (cuda_model.cu:535-540); a library
// GEMM tiles for large m and, at m = 64, streams the weights at a fraction of
// HBM bandwidth (measured with rocBLAS and hipBLASLt on MI355X: 0.4-4 TB/s for
// the TinyLlama projections). Here the weight bytes are the whole cost, so the
// kernel is shaped around reading W once, with every load in flight early:
//   * a workgroup (4 waves) owns 64 output features (W rows) and a range of
//     k; each wave takes a quarter of that range and computes all 64
//     features x all tokens on the 16x16x32 bf16 MFMA (A = 16 W rows x 32 k,
//     straight from memory, 16 bytes per lane; B = X^T, 16 tokens x 32 k, also
//     16 bytes per lane, from L2, where the few-hundred-KB X stays resident);
//   * a wave handles its k range in steps of 128: all of a step's W and X
//     loads are issued before its first MFMA;
//   * the four waves' accumulators are summed through LDS (each wave finishes
//     one 16-feature tile); with k split over several workgroups
//     ("splits"), each stores its partial and the last to arrive on the
//     block's counter sums the partials in split order (so results do not
//     depend on arrival order) and applies the epilogue. A block's splits
//     are placed on one XCD (workgroup ids equal modulo 8), so partials go
//     through that XCD's L2, under the same co-location check as the
//     attention kernels;
//   * epilogues: store (bf16, or fp32 for logits), or the SiLU-gated product
//     of a fused gate|up projection (W = [gate; up], n = 2 * inter): a block
//     owns 32 gate rows and the 32 matching up rows, and writes
//     act[t][j] = silu(g) * u, with g and u first rounded to bf16 as a stored
//     gate|up row would be (the same values silu_mul_split computes from a
//     bf16 GEMM output).
#include <float.h>

#include "../le_common.h"
#include "../le_internal.h"
#include "weight_gemm.h"

namespace le::engine {
namespace {

constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;
constexpr int kFeat = 64;    // W rows per workgroup
constexpr int kStep = 128;   // k per wave step (4 MFMA k-pieces of 32)
constexpr int kTargetWorkgroups = 512;

struct GemmArgs {
  const bf16_t* x;
  const bf16_t* w;
  void* out;
  float* partials;      // [n_blocks][splits][kWaves][MT][64 lanes] f32x4
  arrival_t* counters;  // [n_blocks], zero between launches
  int32_t* misplaced;
  int m, k;
  int inter;            // SiLU epilogue: gate rows (= output columns); else 0
  int out_cols;         // output row stride
  int n_blocks, blocks_pad, splits, steps;
  int out_f32;
  int l2_local;
};

template <int MT>
struct GemmSmem {
  f32x4 red[kWaves][kWaves][MT][kWave];  // [wave][tile][token tile][lane]
  int last;
};

__device__ __forceinline__ bf16x8 ld_bf16x8(const bf16_t* p) { return __builtin_bit_cast(bf16x8, ld16(p)); }

// W row of tile t (16 rows) for lane row r in block b.
__device__ __forceinline__ int64_t w_row(const GemmArgs& a, int b, int t, int r) {
  if (a.inter == 0) return static_cast<int64_t>(b) * kFeat + t * 16 + r;
  const int f = t * 16 + r;  // 0..31 gate, 32..63 up
  return f < 32 ? static_cast<int64_t>(b) * 32 + f : a.inter + static_cast<int64_t>(b) * 32 + (f - 32);
}

template <int MT>
__global__ __launch_bounds__(kThreads) void weight_gemm_kernel(GemmArgs a) {
  __shared__ GemmSmem<MT> sm;
  const int g_id = blockIdx.x;
  const int b = g_id % a.blocks_pad;
  const int split = g_id / a.blocks_pad;
  if (b >= a.n_blocks) return;  // padding of the XCD placement
  const int lane = threadIdx.x % kWave, wv = threadIdx.x / kWave;
  const int r = lane % 16, g = lane / 16;

  // this wave's steps: sub-range q of Q = splits * kWaves equal parts
  const int Q = a.splits * kWaves, q = split * kWaves + wv;
  const int s_begin = static_cast<int>(static_cast<int64_t>(q) * a.steps / Q);
  const int s_end = static_cast<int>(static_cast<int64_t>(q + 1) * a.steps / Q);

  const bf16_t* wp[4];
#pragma unroll
  for (int t = 0; t < 4; t++) wp[t] = a.w + w_row(a, b, t, r) * a.k + 8 * g;
  const bf16_t* xp[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) xp[mt] = a.x + static_cast<int64_t>(min(mt * 16 + r, a.m - 1)) * a.k + 8 * g;

  f32x4 acc[4][MT];
#pragma unroll
  for (int t = 0; t < 4; t++)
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int s = s_begin; s < s_end; s++) {
    const int k0 = s * kStep;
    bf16x8 wa[4][4], xb[MT][4];
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
      for (int j = 0; j < 4; j++) wa[t][j] = ld_bf16x8(wp[t] + k0 + 32 * j);
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int j = 0; j < 4; j++) xb[mt][j] = ld_bf16x8(xp[mt] + k0 + 32 * j);
    // every load of the step is issued before the first MFMA waits on one
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int t = 0; t < 4; t++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
          acc[t][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa[t][j], xb[mt][j], acc[t][mt], 0, 0, 0);
  }

  // The four waves' sums: wave wv finishes tile wv (features 16 wv + 4 g + i,
  // token mt * 16 + r in lane (r, g) of token tile mt).
#pragma unroll
  for (int t = 0; t < 4; t++)
#pragma unroll
    for (int mt = 0; mt < MT; mt++) sm.red[wv][t][mt][lane] = acc[t][mt];
  __syncthreads();
  f32x4 res[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    res[mt] = sm.red[0][wv][mt][lane];
#pragma unroll
    for (int w2 = 1; w2 < kWaves; w2++) res[mt] += sm.red[w2][wv][mt][lane];
  }

  if (a.splits > 1) {
    // store this split's partial, arrive; the last arriver sums all splits
    const int64_t rec = ((static_cast<int64_t>(b) * a.splits + split) * kWaves + wv) * MT;
    const __amdgpu_buffer_rsrc_t rs = coherent_rsrc(a.partials + rec * kWave * 4);
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
      const uint32_t off = static_cast<uint32_t>((mt * kWave + lane) * 16);
      const f32x4v v = __builtin_bit_cast(f32x4v, res[mt]);
      if (a.l2_local) st_l2_16(rs, off, v);
      else st_coherent16(rs, off, v);
    }
    const int rot = a.l2_local ? xcd_rotation(a.l2_local, g_id) : 0;
    __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores are performed
    __syncthreads();                // ... and every other thread's
    if (threadIdx.x == 0) {
      const arrival_t mine = arrival_token(rot);
      const arrival_t seen = __hip_atomic_fetch_add(a.counters + b, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const bool last = arrival_count(seen) == a.splits - 1;
      // partials left in another XCD's L2 are out of reach: poison the block
      const bool apart = last && a.l2_local && !arrivals_colocated(seen + mine, rot);
      if (apart) __hip_atomic_fetch_add(a.misplaced, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sm.last = !last ? 0 : (apart ? 2 : 1);
    }
    __syncthreads();
    if (!sm.last) return;
    const bool poison = sm.last == 2;
    // every other split arrived after its partial was performed
    const int64_t rec0 = static_cast<int64_t>(b) * a.splits * kWaves * MT;
    const __amdgpu_buffer_rsrc_t r0 = coherent_rsrc(a.partials + rec0 * kWave * 4);
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
      f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
      for (int s2 = 0; s2 < a.splits; s2++) {
        f32x4 v;
        if (s2 == split) {
          v = res[mt];
        } else {
          const uint32_t off = static_cast<uint32_t>((((s2 * kWaves + wv) * MT + mt) * kWave + lane) * 16);
          v = __builtin_bit_cast(f32x4, ld_coherent16(r0, off));
        }
        sum += v;
      }
      res[mt] = poison ? f32x4{__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""), __builtin_nanf("")}
                       : sum;
    }
    if (threadIdx.x == 0) __hip_atomic_store(a.counters + b, arrival_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  if (a.inter == 0) {
    const int col = b * kFeat + wv * 16 + 4 * g;
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
      const int tok = mt * 16 + r;
      if (tok >= a.m) continue;
      const float v[4] = {res[mt][0], res[mt][1], res[mt][2], res[mt][3]};
      const int64_t o = static_cast<int64_t>(tok) * a.out_cols + col;
      if (a.out_f32) elem<float>::store4(static_cast<float*>(a.out) + o, v);
      else elem<bf16_t>::store4(static_cast<bf16_t*>(a.out) + o, v);
    }
    return;
  }
  // SiLU-gated product: waves 2, 3 hold the up rows matching waves 0, 1's
  // gate rows; they hand them over through LDS.
  __syncthreads();  // every wave is done reading sm.red
  if (wv >= 2) {
#pragma unroll
    for (int mt = 0; mt < MT; mt++) sm.red[0][wv - 2][mt][lane] = res[mt];
  }
  __syncthreads();
  if (wv >= 2) return;
  const int col = b * 32 + wv * 16 + 4 * g;
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    const int tok = mt * 16 + r;
    if (tok >= a.m) continue;
    const f32x4 u = sm.red[0][wv][mt][lane];
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float gi = elem<bf16_t>::round(res[mt][i]), ui = elem<bf16_t>::round(u[i]);
      v[i] = gi / (1.0f + expf(-gi)) * ui;
    }
    elem<bf16_t>::store4(static_cast<bf16_t*>(a.out) + static_cast<int64_t>(tok) * a.out_cols + col, v);
  }
}

struct Shape {
  int n_blocks, blocks_pad, splits, steps;
  size_t partial_bytes, counter_bytes;
};

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

bool shape_of(int m, int k, int n, bool silu, int splits_req, Shape* sh) {
  if (m < 1 || m > kMaxGemmRows || k <= 0 || k % kStep != 0 || n <= 0) return false;
  if (silu ? (n % 2 != 0 || (n / 2) % 32 != 0) : n % kFeat != 0) return false;
  sh->n_blocks = silu ? n / 2 / 32 : n / kFeat;
  sh->steps = k / kStep;
  int s = splits_req > 0 ? splits_req : (kTargetWorkgroups + sh->n_blocks - 1) / sh->n_blocks;
  const int max_s = sh->steps / kWaves;  // every wave keeps at least one step
  if (s > max_s) s = max_s;
  if (s < 1) s = 1;
  sh->splits = s;
  sh->blocks_pad = s > 1 ? (sh->n_blocks + 7) / 8 * 8 : sh->n_blocks;
  const int mt = (m + 15) / 16;
  sh->counter_bytes = align_up(static_cast<size_t>(sh->n_blocks) * 8);
  sh->partial_bytes = s > 1 ? static_cast<size_t>(sh->n_blocks) * s * kWaves * mt * kWave * 16 : 0;
  return true;
}

}  // namespace

bool weight_gemm_supported(int m, int k, int n, bool silu) {
  Shape sh;
  return shape_of(m, k, n, silu, 0, &sh);
}

size_t weight_gemm_workspace(int m, int k, int n, bool silu, int splits) {
  Shape sh;
  if (!shape_of(m, k, n, silu, splits, &sh)) return 0;
  return sh.splits > 1 ? sh.counter_bytes + sh.partial_bytes : 0;
}

hipError_t weight_gemm(const void* x, int m, int k, const void* w, int n, bool silu, void* out, bool out_f32,
                       void* ws, size_t ws_bytes, int splits, hipStream_t s) {
  Shape sh;
  if (!shape_of(m, k, n, silu, splits, &sh) || (silu && out_f32)) return hipErrorInvalidValue;
  GemmArgs a{};
  a.x = static_cast<const bf16_t*>(x);
  a.w = static_cast<const bf16_t*>(w);
  a.out = out;
  a.m = m;
  a.k = k;
  a.inter = silu ? n / 2 : 0;
  a.out_cols = silu ? n / 2 : n;
  a.n_blocks = sh.n_blocks;
  a.blocks_pad = sh.blocks_pad;
  a.splits = sh.splits;
  a.steps = sh.steps;
  a.out_f32 = out_f32 ? 1 : 0;
  if (sh.splits > 1) {
    if (!ws || ws_bytes < sh.counter_bytes + sh.partial_bytes) return hipErrorInvalidValue;
    a.counters = static_cast<arrival_t*>(ws);
    a.partials = reinterpret_cast<float*>(static_cast<char*>(ws) + sh.counter_bytes);
    a.l2_local = xcd_placement_holds(s) ? 1 : 0;
    if (a.l2_local) a.misplaced = xcd_miss_counter();
    if (!a.misplaced) a.l2_local = 0;
  }
  const dim3 grid(static_cast<unsigned>(sh.splits * sh.blocks_pad));
  switch ((m + 15) / 16) {
    case 1: weight_gemm_kernel<1><<<grid, kThreads, 0, s>>>(a); break;
    case 2: weight_gemm_kernel<2><<<grid, kThreads, 0, s>>>(a); break;
    case 3: weight_gemm_kernel<3><<<grid, kThreads, 0, s>>>(a); break;
    default: weight_gemm_kernel<4><<<grid, kThreads, 0, s>>>(a); break;
  }
  return hipGetLastError();
}

}  // namespace le::engine
