// Layer kernels around the attention path for the device model: embedding
// gather, RMSNorm, RoPE, SiLU-gated product, residual and bias adds, logit-row
// gather and greedy argmax. Each restates one reference op (ops.h, the CUDA
// kernels in src/kernels/) for fp32 or bf16 activations; the math is fp32.
#include <float.h>

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

// out[r] = x[r] * rsqrt(mean(x[r]^2) + eps) * w (ops.h:22-31); one workgroup per row,
// fp32 sum of squares.
template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const T* __restrict__ x, const float* __restrict__ w,
                                                      T* __restrict__ out, int cols, float eps) {
  const T* xr = x + static_cast<int64_t>(blockIdx.x) * cols;
  T* o = out + static_cast<int64_t>(blockIdx.x) * cols;
  float ss = 0.f;
  for (int j = threadIdx.x; j < cols; j += 256) {
    const float v = ld(xr + j);
    ss += v * v;
  }
  __shared__ float part[4];
  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = (part[0] + part[1]) + (part[2] + part[3]);
  const float inv = 1.0f / sqrtf(tot / cols + eps);
  for (int j = threadIdx.x; j < cols; j += 256) st(o + j, ld(xr + j) * inv * w[j]);
}

// rotate_half RoPE in place on `heads` heads of each row (ops.h:55-66).
template <typename T>
__global__ void rope_kernel(T* __restrict__ x, const int32_t* __restrict__ positions,
                            const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                            int heads, int head_dim, int row_stride) {
  const int half = head_dim / 2;
  const int t = blockIdx.x;
  const int64_t tab = static_cast<int64_t>(positions[t]) * half;
  T* row = x + static_cast<int64_t>(t) * row_stride;
  for (int i = threadIdx.x; i < heads * half; i += blockDim.x) {
    const int h = i / half, k = i - h * half;
    T* v = row + h * head_dim;
    const float c = cos_t[tab + k], s = sin_t[tab + k];
    const float a = ld(v + k), b = ld(v + k + half);
    st(v + k, a * c - b * s);
    st(v + k + half, b * c + a * s);
  }
}

// gate = silu(gate) * up (ops.h:69-74)
template <typename T>
__global__ void silu_mul_kernel(T* __restrict__ gate, const T* __restrict__ up, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const float g = ld(gate + i);
    st(gate + i, g / (1.0f + expf(-g)) * ld(up + i));
  }
}

template <typename T>
__global__ void add_kernel(T* __restrict__ x, const T* __restrict__ y, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    st(x + i, ld(x + i) + ld(y + i));
}

template <typename T>
__global__ void add_bias_kernel(T* __restrict__ x, const float* __restrict__ bias, int cols, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    st(x + i, ld(x + i) + bias[i % cols]);
}

// Greedy token per logits row: the first maximum wins (sampler.cpp:9-13).
// One workgroup per row; each thread keeps its own (max, lowest index), then a
// tree merge that prefers the lower index on ties. NaN never wins (as with the
// reference's strict `>`, a NaN is never greater).
__global__ __launch_bounds__(256) void argmax_kernel(const float* __restrict__ logits, int vocab,
                                                     int32_t* __restrict__ out) {
  const float* row = logits + static_cast<int64_t>(blockIdx.x) * vocab;
  float best = -INFINITY;
  int idx = vocab;  // "none yet"
  for (int j = threadIdx.x; j < vocab; j += 256) {
    const float v = row[j];
    if (v > best || (idx == vocab && v == v)) { best = v; idx = j; }
  }
  __shared__ float sv[256];
  __shared__ int si[256];
  sv[threadIdx.x] = best;
  si[threadIdx.x] = idx;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      const float ov = sv[threadIdx.x + s];
      const int oi = si[threadIdx.x + s];
      const bool take = oi < vocab && (si[threadIdx.x] == vocab || ov > sv[threadIdx.x] ||
                                       (ov == sv[threadIdx.x] && oi < si[threadIdx.x]));
      if (take) { sv[threadIdx.x] = ov; si[threadIdx.x] = oi; }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) out[blockIdx.x] = si[0] == vocab ? 0 : si[0];
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

hipError_t rmsnorm(const void* x, const float* w, void* out, int rows, int cols, float eps, bool bf16,
                   hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  LE_DISPATCH(bf16, rmsnorm_kernel<T><<<rows, 256, 0, s>>>(static_cast<const T*>(x), w,
                                                           static_cast<T*>(out), cols, eps));
  return hipGetLastError();
}

hipError_t rope(void* x, const int32_t* positions, const float* cos_t, const float* sin_t, int n,
                int heads, int head_dim, int row_stride, bool bf16, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  LE_DISPATCH(bf16, rope_kernel<T><<<n, 256, 0, s>>>(static_cast<T*>(x), positions, cos_t, sin_t,
                                                      heads, head_dim, row_stride));
  return hipGetLastError();
}

hipError_t silu_mul(void* gate, const void* up, int64_t n, bool bf16, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  LE_DISPATCH(bf16, silu_mul_kernel<T><<<grid_for(n), 256, 0, s>>>(static_cast<T*>(gate),
                                                                    static_cast<const T*>(up), n));
  return hipGetLastError();
}

hipError_t add_inplace(void* x, const void* y, int64_t n, bool bf16, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  LE_DISPATCH(bf16, add_kernel<T><<<grid_for(n), 256, 0, s>>>(static_cast<T*>(x),
                                                               static_cast<const T*>(y), n));
  return hipGetLastError();
}

hipError_t add_bias(void* x, const float* bias, int rows, int cols, bool bf16, hipStream_t s) {
  const int64_t n = static_cast<int64_t>(rows) * cols;
  if (n <= 0) return hipSuccess;
  LE_DISPATCH(bf16, add_bias_kernel<T><<<grid_for(n), 256, 0, s>>>(static_cast<T*>(x), bias, cols, n));
  return hipGetLastError();
}

hipError_t argmax_rows(const float* logits, int rows, int vocab, int32_t* out, hipStream_t s) {
  if (rows <= 0) return hipSuccess;
  argmax_kernel<<<rows, 256, 0, s>>>(logits, vocab, out);
  return hipGetLastError();
}

}  // namespace le::engine
