// Layer kernels around the attention path for the device model: embedding
// gather, residual add + RMSNorm (optionally over gathered logit rows), the
// SiLU-gated product and greedy argmax. Bias and RoPE are fused into the K/V
// cache write (rope_kv_write.hip). Each restates one reference op (ops.h, the CUDA
// kernels in src/kernels/) for fp32 or bf16 activations; the math is fp32.
#include <float.h>

#include <algorithm>

#include "../le_common.h"
#include "model_kernels.h"

namespace le::engine {
namespace {

template <typename T> __device__ __forceinline__ float ld(const T* p);
template <> __device__ __forceinline__ float ld<float>(const float* p) { return *p; }
template <> __device__ __forceinline__ float ld<bf16_t>(const bf16_t* p) { return elem<bf16_t>::load1(p); }
template <typename T> __device__ __forceinline__ void st(T* p, float v);
template <> __device__ __forceinline__ void st<float>(float* p, float v) { *p = v; }
template <> __device__ __forceinline__ void st<bf16_t>(bf16_t* p, float v) { elem<bf16_t>::store1(p, v); }

// out[t] = table[ids[t]] (embedding.cu:9-29)
template <typename T>
__global__ void gather_rows_kernel(const T* __restrict__ table, const int32_t* __restrict__ ids,
                                   T* __restrict__ out, int cols) {
  const int64_t src = static_cast<int64_t>(ids[blockIdx.x]) * cols;
  const int64_t dst = static_cast<int64_t>(blockIdx.x) * cols;
  for (int j = threadIdx.x; j < cols; j += blockDim.x) out[dst + j] = table[src + j];
}

// Residual add fused with the RMSNorm that follows it: cuda_model.cu:381+384,
// 390 + the next layer's 353, and 390 + the head's 404-409 (only the logit
// rows are added and normalised there).
// Output row b reads source row r = rows ? rows[b] : b; v = x[r] + y[r] rounded to T as the separate add
// stores it, written back to x[r] when write_x; out[b] = rmsnorm(v) * w with
// a thread-strided fp32 sum of squares reduced per wave, then across the
// four waves. y == nullptr is a plain norm.
template <typename T>
__global__ __launch_bounds__(256) void residual_rmsnorm_kernel(T* __restrict__ x, const T* __restrict__ y,
                                                               const int32_t* __restrict__ rows,
                                                               const float* __restrict__ w,
                                                               T* __restrict__ out, int cols, float eps,
                                                               int write_x) {
  const int64_t r = rows ? rows[blockIdx.x] : blockIdx.x;
  T* xr = x + r * cols;
  const T* yr = y ? y + r * cols : nullptr;
  T* o = out + static_cast<int64_t>(blockIdx.x) * cols;
  float ss = 0.f;
  for (int j = threadIdx.x; j < cols; j += 256) {
    float v = ld(xr + j);
    if (yr) {
      T tmp;
      st(&tmp, v + ld(yr + j));
      v = ld(&tmp);
      if (write_x) xr[j] = tmp;
    }
    ss += v * v;
  }
  __shared__ float part[4];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = (part[0] + part[1]) + (part[2] + part[3]);
  const float inv = 1.0f / sqrtf(tot / cols + eps);
  for (int j = threadIdx.x; j < cols; j += 256) {
    float v;
    if (yr && write_x) {
      v = ld(xr + j);  // this thread's own store above
    } else if (yr) {
      T tmp;
      st(&tmp, ld(xr + j) + ld(yr + j));
      v = ld(&tmp);
    } else {
      v = ld(xr + j);
    }
    st(o + j, v * inv * w[j]);
  }
}

// Vector form of residual_rmsnorm_kernel for rows of at most 4 x 256 x VEC
// elements with cols % VEC == 0 (VEC = elements per 16 bytes): each thread
// loads its pieces of x and y with 16-byte accesses, keeps the row in
// registers between the sum of squares and the scaling, and stores with
// 16-byte accesses. Same rounding of the residual sum as the scalar kernel;
// the sum of squares is accumulated per thread over its pieces in order,
// then reduced per wave and across the four waves.
template <typename T> struct vec16;
template <> struct vec16<float> {
  static constexpr int N = 4;
  __device__ __forceinline__ static void load(const float* p, float* o) {
    const float4 r = *reinterpret_cast<const float4*>(p);
    o[0] = r.x; o[1] = r.y; o[2] = r.z; o[3] = r.w;
  }
  __device__ __forceinline__ static void store(float* p, const float* v) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
  __device__ __forceinline__ static float round(float x) { return x; }
};
template <> struct vec16<bf16_t> {
  static constexpr int N = 8;
  __device__ __forceinline__ static void load(const bf16_t* p, float* o) { elem<bf16_t>::widen(ld16(p), o); }
  __device__ __forceinline__ static void store(bf16_t* p, const float* v) {
    *reinterpret_cast<uint4*>(p) = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                              pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
  }
  __device__ __forceinline__ static float round(float x) { return __uint_as_float(f32_to_bf16_bits(x) << 16); }
};

constexpr int kNormPieces = 4;  // 16-byte pieces per thread at most

template <typename T>
__global__ __launch_bounds__(256) void residual_rmsnorm_vec_kernel(T* __restrict__ x, const T* __restrict__ y,
                                                                   const int32_t* __restrict__ rows,
                                                                   const float* __restrict__ w,
                                                                   T* __restrict__ out, int cols, float eps,
                                                                   int write_x) {
  constexpr int V = vec16<T>::N;
  const int64_t r = rows ? rows[blockIdx.x] : blockIdx.x;
  T* xr = x + r * cols;
  const T* yr = y ? y + r * cols : nullptr;
  T* o = out + static_cast<int64_t>(blockIdx.x) * cols;
  const int pieces = cols / V;
  float v[kNormPieces][V];
  float yv[kNormPieces][V];
#pragma unroll
  for (int i = 0; i < kNormPieces; i++) {
    const int pc = threadIdx.x + i * 256;
    if (pc < pieces) {
      vec16<T>::load(xr + pc * V, v[i]);
      if (yr) vec16<T>::load(yr + pc * V, yv[i]);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kNormPieces; i++) {
    const int pc = threadIdx.x + i * 256;
    if (pc < pieces) {
      if (yr) {
#pragma unroll
        for (int e = 0; e < V; e++) v[i][e] = vec16<T>::round(v[i][e] + yv[i][e]);
        if (write_x) vec16<T>::store(xr + pc * V, v[i]);
      }
#pragma unroll
      for (int e = 0; e < V; e++) ss += v[i][e] * v[i][e];
    }
  }
  __shared__ float part[4];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = (part[0] + part[1]) + (part[2] + part[3]);
  const float inv = 1.0f / sqrtf(tot / cols + eps);
#pragma unroll
  for (int i = 0; i < kNormPieces; i++) {
    const int pc = threadIdx.x + i * 256;
    if (pc < pieces) {
      float ov[V];
#pragma unroll
      for (int e = 0; e < V; e++) ov[e] = v[i][e] * inv * w[pc * V + e];
      vec16<T>::store(o + pc * V, ov);
    }
  }
}

// act[t][j] = silu(gu[t][j]) * gu[t][inter + j], 16 bytes of output per
// thread (inter % VEC == 0).
template <typename T>
__global__ void silu_mul_split_vec_kernel(const T* __restrict__ gu, T* __restrict__ act, int inter, int64_t n_pieces) {
  constexpr int V = vec16<T>::N;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n_pieces) return;
  const int per_row = inter / V;
  const int64_t t = i / per_row;
  const int j = static_cast<int>(i - t * per_row) * V;
  const T* row = gu + t * 2 * inter;
  float g[V], u[V], o[V];
  vec16<T>::load(row + j, g);
  vec16<T>::load(row + inter + j, u);
#pragma unroll
  for (int e = 0; e < V; e++) o[e] = g[e] / (1.0f + expf(-g[e])) * u[e];
  vec16<T>::store(act + t * inter + j, o);
}

// The post-attention RMSNorm of the bf16 model folded around its gate|up
// projection: the norm weight w is folded into the projection's input
// columns (gate|up = x . (W diag w)^T, rounded to bf16 once at load), so the
// projection reads the residual stream x itself, and the row's scale
// r = 1/sqrt(mean(x^2) + eps) is applied here to both halves before the SiLU
// product: act[t][j] = silu(g r) * (u r). The residual add before it runs in
// the O projection's epilogue (beta = 1). Workgroup (t, s) takes the s-th of
// S contiguous ranges of row t's pieces of g and u (S = gridDim.y: a decode
// step's few rows spread over more CUs) and forms r itself from the whole
// row of x; x and its
// pieces of g and u are requested together, so a workgroup costs one memory
// round trip. Rows of at most 4 x 256 x 8 elements.
constexpr int kFusedPieces = 4;
__global__ __launch_bounds__(256) void rms_silu_mul_kernel(const bf16_t* __restrict__ x,
                                                          const bf16_t* __restrict__ gu,
                                                          bf16_t* __restrict__ act, int hidden, int inter,
                                                          float eps) {
  constexpr int V = 8;
  const int64_t t = blockIdx.x;
  const bf16_t* xr = x + t * hidden;
  const bf16_t* g_row = gu + t * 2 * inter;
  bf16_t* out = act + t * inter;
  const int hp = hidden / V, ip = inter / V;
  const int chunk = (ip + static_cast<int>(gridDim.y) - 1) / static_cast<int>(gridDim.y);
  const int p0 = static_cast<int>(blockIdx.y) * chunk, p1 = min(ip, p0 + chunk);
  float xv[kFusedPieces][V], g[kFusedPieces][V], u[kFusedPieces][V];
#pragma unroll
  for (int i = 0; i < kFusedPieces; i++) {
    const int px = threadIdx.x + i * 256;
    if (px < hp) vec16<bf16_t>::load(xr + px * V, xv[i]);
    const int pc = p0 + threadIdx.x + i * 256;
    if (pc < p1) {
      vec16<bf16_t>::load(g_row + pc * V, g[i]);
      vec16<bf16_t>::load(g_row + inter + pc * V, u[i]);
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kFusedPieces; i++)
    if (threadIdx.x + i * 256 < hp)
#pragma unroll
      for (int e = 0; e < V; e++) ss += xv[i][e] * xv[i][e];
  __shared__ float part[4];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = (part[0] + part[1]) + (part[2] + part[3]);
  const float r = 1.0f / sqrtf(tot / hidden + eps);
#pragma unroll
  for (int i = 0; i < kFusedPieces; i++) {
    const int pc = p0 + threadIdx.x + i * 256;
    if (pc < p1) {
      float o[V];
#pragma unroll
      for (int e = 0; e < V; e++) {
        const float gv = g[i][e] * r;
        o[e] = gv / (1.0f + expf(-gv)) * (u[i][e] * r);
      }
      vec16<bf16_t>::store(out + pc * V, o);
    }
  }
}

// act[t][j] = silu(gu[t][j]) * gu[t][inter + j]: the SiLU-gated product over
// the fused gate|up projection output (ops.h:69-74, elementwise.cu).
template <typename T>
__global__ void silu_mul_split_kernel(const T* __restrict__ gu, T* __restrict__ act, int inter, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t t = i / inter, j = i - t * inter;
    const T* row = gu + t * 2 * inter;
    const float g = ld(row + j);
    st(act + i, g / (1.0f + expf(-g)) * ld(row + inter + j));
  }
}

// Greedy token per logits row: the first maximum wins (sampler.cpp:9-13).
// One 1024-thread workgroup per row; each thread scans its 16-byte pieces in
// index order keeping (max, lowest index), then the waves and the workgroup
// merge with a rule that prefers the lower index on ties. NaN never wins (as
// with the reference's strict `>`, a NaN is never greater), and a NaN in
// element 0 is never replaced.
constexpr int kArgmaxThreads = 1024;

__device__ __forceinline__ void argmax_take(float& bv, int& bi, float v, int i, int none) {
  if (i < none && (bi == none || v > bv || (v == bv && i < bi))) { bv = v; bi = i; }
}

__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const float* __restrict__ logits, int vocab,
                                                                int32_t* __restrict__ out) {
  const float* row = logits + static_cast<int64_t>(blockIdx.x) * vocab;
  float best = -INFINITY;
  int idx = vocab;  // "none yet"
  auto scan = [&](float v, int j) {
    if (v > best || (idx == vocab && v == v)) { best = v; idx = j; }
  };
  if (vocab % 4 == 0) {
    const float4* r4 = reinterpret_cast<const float4*>(row);
    for (int j4 = threadIdx.x; j4 < vocab / 4; j4 += kArgmaxThreads) {
      const float4 v = r4[j4];
      scan(v.x, 4 * j4); scan(v.y, 4 * j4 + 1); scan(v.z, 4 * j4 + 2); scan(v.w, 4 * j4 + 3);
    }
  } else {
    for (int j = threadIdx.x; j < vocab; j += kArgmaxThreads) scan(row[j], j);
  }
  // a thread's candidate has the lowest index among its equal maxima; merge
  // across lanes, then across the waves
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(best, off, kWave);
    const int oi = __shfl_xor(idx, off, kWave);
    argmax_take(best, idx, ov, oi, vocab);
  }
  __shared__ float sv[kArgmaxThreads / kWave];
  __shared__ int si[kArgmaxThreads / kWave];
  const int wave = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) {
    sv[wave] = best;
    si[wave] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float bv = sv[0];
    int bi = si[0];
    for (int w = 1; w < kArgmaxThreads / kWave; w++) argmax_take(bv, bi, sv[w], si[w], vocab);
    // the reference starts from element 0 and replaces it only by a greater
    // value, so a NaN there is never replaced
    out[blockIdx.x] = (bi == vocab || row[0] != row[0]) ? 0 : bi;
  }
}

int grid_for(int64_t n) {
  const int64_t b = (n + 255) / 256;
  return static_cast<int>(b < 4096 ? (b > 0 ? b : 1) : 4096);
}

}  // namespace

#define LE_DISPATCH(bf16, ...) \
  do { if (bf16) { using T = bf16_t; __VA_ARGS__; } else { using T = float; __VA_ARGS__; } } while (0)

hipError_t gather_rows(const void* table, const int32_t* ids, void* out, int n, int cols, bool bf16,
                       hipStream_t s) {
  if (n <= 0) return hipSuccess;
  LE_DISPATCH(bf16, gather_rows_kernel<T><<<n, 256, 0, s>>>(static_cast<const T*>(table), ids,
                                                             static_cast<T*>(out), cols));
  return hipGetLastError();
}

hipError_t residual_rmsnorm(void* x, const void* y, const int32_t* rows, const float* w, void* out,
                            int n_out, int cols, float eps, bool write_x, bool bf16, hipStream_t s) {
  if (n_out <= 0) return hipSuccess;
  const int V = bf16 ? 8 : 4;
  const bool aligned = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                         reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(w)) & 15) == 0;
  if (aligned && cols % V == 0 && cols <= 256 * V * kNormPieces) {
    LE_DISPATCH(bf16, residual_rmsnorm_vec_kernel<T><<<n_out, 256, 0, s>>>(
                          static_cast<T*>(x), static_cast<const T*>(y), rows, w, static_cast<T*>(out), cols,
                          eps, write_x ? 1 : 0));
    return hipGetLastError();
  }
  LE_DISPATCH(bf16, residual_rmsnorm_kernel<T><<<n_out, 256, 0, s>>>(
                        static_cast<T*>(x), static_cast<const T*>(y), rows, w, static_cast<T*>(out), cols,
                        eps, write_x ? 1 : 0));
  return hipGetLastError();
}

bool rms_silu_mul_fits(int hidden, int inter) {
  return hidden % 8 == 0 && inter % 8 == 0 && hidden <= kFusedPieces * 256 * 8 && inter <= kFusedPieces * 256 * 8;
}

hipError_t rms_silu_mul(const void* x, const void* gate_up, void* act, int rows, int hidden, int inter, float eps,
                        hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  if (!rms_silu_mul_fits(hidden, inter) ||
      ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gate_up) | reinterpret_cast<uintptr_t>(act)) &
       15) != 0)
    return hipErrorInvalidValue;
  // pieces of a row per workgroup: a decode step's rows spread over about 256
  // workgroups (each re-reads its row of x, a few KB)
  const int S = std::max(1, std::min(8, 256 / rows));
  rms_silu_mul_kernel<<<dim3(static_cast<unsigned>(rows), static_cast<unsigned>(S)), 256, 0, s>>>(
      static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(gate_up), static_cast<bf16_t*>(act), hidden, inter,
      eps);
  return hipGetLastError();
}

hipError_t silu_mul_split(const void* gate_up, void* act, int rows, int inter, bool bf16, hipStream_t s) {
  const int64_t n = static_cast<int64_t>(rows) * inter;
  if (n <= 0) return hipSuccess;
  const int V = bf16 ? 8 : 4;
  if (inter % V == 0 && ((reinterpret_cast<uintptr_t>(gate_up) | reinterpret_cast<uintptr_t>(act)) & 15) == 0) {
    const int64_t pieces = n / V;
    LE_DISPATCH(bf16, silu_mul_split_vec_kernel<T><<<static_cast<unsigned>((pieces + 255) / 256), 256, 0, s>>>(
                          static_cast<const T*>(gate_up), static_cast<T*>(act), inter, pieces));
    return hipGetLastError();
  }
  LE_DISPATCH(bf16, silu_mul_split_kernel<T><<<grid_for(n), 256, 0, s>>>(
                        static_cast<const T*>(gate_up), static_cast<T*>(act), inter, n));
  return hipGetLastError();
}

hipError_t argmax_rows(const float* logits, int rows, int vocab, int32_t* out, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  argmax_kernel<<<rows, kArgmaxThreads, 0, s>>>(logits, vocab, out);
  return hipGetLastError();
}

}  // namespace le::engine
