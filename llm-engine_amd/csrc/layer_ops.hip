// The reference's small per-layer kernels, behind the C ABI for any element
// type (fp32, bf16, fp16): embedding gather, RMSNorm, SiLU-gated product,
// RoPE, residual add and bias add (cuda_kernels.h:17-40, the launchers that
// cuda_model.cu:347-390 calls between the GEMMs and attention). The device
// model fuses these into fewer launches (model_kernels.hip, rope_kv_write.hip);
// these entry points exist so the reference engine's own call sequence runs
// on this library unchanged (the bridge, le_cuda_kernels.h).
//
// Arithmetic is fp32 with one rounding to the element type per stored value,
// as the reference kernels do. Bit-exact with the oracle: embedding, residual
// and bias adds, RoPE (no contraction: a*c - b*s rounded once). RMSNorm and
// SiLU differ from the CPU only in the order of the sum of squares and in
// expf's last bits, before the output's rounding.
#include <float.h>

#include "le_common.h"
#include "llm_engine_amd.h"

namespace le {
namespace {

constexpr int kThreads = 256;

int grid_for(int64_t work_items) {
  const int64_t b = (work_items + kThreads - 1) / kThreads;
  return static_cast<int>(b < 4096 ? (b > 0 ? b : 1) : 4096);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// out[t] = table[ids[t]] (embedding.cu:9-29): raw element copies, 16 bytes
// per thread where rows allow it.
template <typename T>
__global__ __launch_bounds__(kThreads) void embedding_kernel(const T* __restrict__ table, const int32_t* __restrict__ ids,
                                                             T* __restrict__ out, int hidden, int vec) {
  const int64_t src = static_cast<int64_t>(ids[blockIdx.x]) * hidden;
  const int64_t dst = static_cast<int64_t>(blockIdx.x) * hidden;
  if (vec) {
    constexpr int V = 16 / sizeof(T);
    for (int j = threadIdx.x * V; j < hidden; j += kThreads * V)
      *reinterpret_cast<uint4*>(out + dst + j) = *reinterpret_cast<const uint4*>(table + src + j);
  } else {
    for (int j = threadIdx.x; j < hidden; j += kThreads) out[dst + j] = table[src + j];
  }
}

// out[r] = x[r] * 1/sqrt(mean(x[r]^2) + eps) * w (rmsnorm.cu:72-103, ops.h:22-35):
// one workgroup per row, a per-thread fp32 sum of squares reduced per wave and
// across the four waves.
template <typename T>
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const T* __restrict__ x, const float* __restrict__ w,
                                                           T* __restrict__ out, int cols, float eps) {
  const T* xr = x + static_cast<int64_t>(blockIdx.x) * cols;
  T* o = out + static_cast<int64_t>(blockIdx.x) * cols;
  float ss = 0.f;
  for (int j = threadIdx.x; j < cols; j += kThreads) {
    const float v = elem<T>::load1(xr + j);
    ss += v * v;
  }
  __shared__ float part[kThreads / kWave];
  ss = wave_sum(ss);
  if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = ss;
  __syncthreads();
  const float tot = (part[0] + part[1]) + (part[2] + part[3]);
  const float inv = 1.0f / sqrtf(tot / static_cast<float>(cols) + eps);
  for (int j = threadIdx.x; j < cols; j += kThreads) elem<T>::store1(o + j, elem<T>::load1(xr + j) * inv * w[j]);
}

// gate[i] = silu(gate[i]) * up[i] in place (silu_mul.cu:15-23, ops.h:69-74),
// eight elements per thread when vec.
template <typename T>
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(T* __restrict__ gate, const T* __restrict__ up,
                                                            int64_t n, int vec) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (vec) {
    for (int64_t i = i0 * 8; i < n; i += stride * 8) {
      float g[8], u[8];
      elem<T>::load8(gate + i, g);
      elem<T>::load8(up + i, u);
#pragma unroll
      for (int e = 0; e < 8; e++) g[e] = g[e] / (1.0f + expf(-g[e])) * u[e];
      elem<T>::store8(gate + i, g);
    }
  } else {
    for (int64_t i = i0; i < n; i += stride) {
      const float g = elem<T>::load1(gate + i);
      elem<T>::store1(gate + i, g / (1.0f + expf(-g)) * elem<T>::load1(up + i));
    }
  }
}

// x[i] += y[i] (elementwise.cu:20-25) or x[r][c] += bias[c] (elementwise.cu:29-35),
// one rounding to T per element.
template <typename T, bool BIAS>
__global__ __launch_bounds__(kThreads) void add_kernel(T* __restrict__ x, const T* __restrict__ y,
                                                       const float* __restrict__ bias, int64_t n, int cols, int vec) {
#pragma clang fp contract(off)
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (vec) {  // cols % 8 == 0 with a bias
    for (int64_t i = i0 * 8; i < n; i += stride * 8) {
      float a[8], b[8];
      elem<T>::load8(x + i, a);
      if constexpr (BIAS) {
        const int c = static_cast<int>(i % cols);
#pragma unroll
        for (int e = 0; e < 8; e++) b[e] = bias[c + e];
      } else {
        elem<T>::load8(y + i, b);
      }
#pragma unroll
      for (int e = 0; e < 8; e++) a[e] = a[e] + b[e];
      elem<T>::store8(x + i, a);
    }
  } else {
    for (int64_t i = i0; i < n; i += stride) {
      const float b = BIAS ? bias[i % cols] : elem<T>::load1(y + i);
      elem<T>::store1(x + i, elem<T>::load1(x + i) + b);
    }
  }
}

// Rotary embedding in place, rotate_half pairing (rope.cu:33-52, ops.h:52-66):
// x[i] = a*c - b*s, x[i+half] = b*c + a*s with a = x[i], b = x[i+half], no
// contraction, one workgroup per token covering its heads' pairs. Tokens
// whose position is outside [0, max_pos) (max_pos > 0) are left unchanged.
template <typename T>
__global__ __launch_bounds__(kThreads) void rope_kernel(T* __restrict__ x, const int32_t* __restrict__ positions,
                                                        const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                                                        int heads, int head_dim, int row_stride, int max_pos) {
#pragma clang fp contract(off)
  const int pos = positions[blockIdx.x];
  if (pos < 0 || (max_pos > 0 && pos >= max_pos)) return;
  const int half = head_dim / 2;
  T* row = x + static_cast<int64_t>(blockIdx.x) * row_stride;
  const float* c = cos_t + static_cast<int64_t>(pos) * half;
  const float* s = sin_t + static_cast<int64_t>(pos) * half;
  for (int k = threadIdx.x; k < heads * half; k += kThreads) {
    const int h = k / half, i = k - h * half;
    T* v = row + h * head_dim;
    const float a = elem<T>::load1(v + i), b = elem<T>::load1(v + i + half);
    const float ci = c[i], si = s[i];
    const float lo = a * ci - b * si;
    const float hi = b * ci + a * si;
    elem<T>::store1(v + i, lo);
    elem<T>::store1(v + i + half, hi);
  }
}

bool valid_dtype(le_dtype d) { return d == LE_F32 || d == LE_BF16 || d == LE_F16; }

int status(hipError_t e) { return e == hipSuccess ? LE_OK : static_cast<int>(e); }

}  // namespace
}  // namespace le

using le::with_dtype;

extern "C" {

int le_embedding(const void* table, le_dtype dtype, const int32_t* ids, void* out, int n_tokens, int hidden,
                 hipStream_t stream) {
  if (n_tokens < 0 || hidden < 0 || !le::valid_dtype(dtype)) return LE_EINVAL;
  if (n_tokens == 0 || hidden == 0) return LE_OK;
  if (!table || !ids || !out) return LE_EINVAL;
  return le::status(with_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    const int vec = (hidden * static_cast<int>(sizeof(T))) % 16 == 0 && le::aligned16(table) && le::aligned16(out);
    le::embedding_kernel<T><<<n_tokens, le::kThreads, 0, stream>>>(static_cast<const T*>(table), ids,
                                                                    static_cast<T*>(out), hidden, vec);
    return hipGetLastError();
  }));
}

int le_rmsnorm(const void* x, le_dtype dtype, const float* weight, void* out, int rows, int cols, float eps,
               hipStream_t stream) {
  if (rows < 0 || cols < 0 || !le::valid_dtype(dtype)) return LE_EINVAL;
  if (rows == 0 || cols == 0) return LE_OK;
  if (!x || !weight || !out) return LE_EINVAL;
  return le::status(with_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    le::rmsnorm_kernel<T><<<rows, le::kThreads, 0, stream>>>(static_cast<const T*>(x), weight, static_cast<T*>(out),
                                                              cols, eps);
    return hipGetLastError();
  }));
}

int le_silu_mul(void* gate, const void* up, le_dtype dtype, size_t n, hipStream_t stream) {
  if (!le::valid_dtype(dtype) || n > (size_t{1} << 62)) return LE_EINVAL;
  if (n == 0) return LE_OK;
  if (!gate || !up) return LE_EINVAL;
  return le::status(with_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    const int vec = n % 8 == 0 && le::aligned16(gate) && le::aligned16(up);
    const int64_t items = vec ? static_cast<int64_t>(n / 8) : static_cast<int64_t>(n);
    le::silu_mul_kernel<T><<<le::grid_for(items), le::kThreads, 0, stream>>>(
        static_cast<T*>(gate), static_cast<const T*>(up), static_cast<int64_t>(n), vec);
    return hipGetLastError();
  }));
}

int le_add_inplace(void* x, const void* y, le_dtype dtype, size_t n, hipStream_t stream) {
  if (!le::valid_dtype(dtype) || n > (size_t{1} << 62)) return LE_EINVAL;
  if (n == 0) return LE_OK;
  if (!x || !y) return LE_EINVAL;
  return le::status(with_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    const int vec = n % 8 == 0 && le::aligned16(x) && le::aligned16(y);
    const int64_t items = vec ? static_cast<int64_t>(n / 8) : static_cast<int64_t>(n);
    le::add_kernel<T, false><<<le::grid_for(items), le::kThreads, 0, stream>>>(
        static_cast<T*>(x), static_cast<const T*>(y), nullptr, static_cast<int64_t>(n), 1, vec);
    return hipGetLastError();
  }));
}

int le_add_bias(void* x, le_dtype dtype, const float* bias, int rows, int cols, hipStream_t stream) {
  if (rows < 0 || cols < 0 || !le::valid_dtype(dtype)) return LE_EINVAL;
  if (rows == 0 || cols == 0) return LE_OK;
  if (!x || !bias) return LE_EINVAL;
  const int64_t n = static_cast<int64_t>(rows) * cols;
  return le::status(with_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    const int vec = cols % 8 == 0 && le::aligned16(x);
    le::add_kernel<T, true><<<le::grid_for(vec ? n / 8 : n), le::kThreads, 0, stream>>>(
        static_cast<T*>(x), nullptr, bias, n, cols, vec);
    return hipGetLastError();
  }));
}

int le_rope(void* x, le_dtype dtype, const int32_t* positions, const float* cos_table, const float* sin_table,
            int max_pos, int n_tokens, int heads, int head_dim, int row_stride, hipStream_t stream) {
  if (n_tokens < 0 || heads < 0 || head_dim < 0 || head_dim % 2 != 0 || !le::valid_dtype(dtype)) return LE_EINVAL;
  if (n_tokens == 0 || heads == 0 || head_dim == 0) return LE_OK;
  if (!x || !positions || !cos_table || !sin_table || row_stride < heads * head_dim) return LE_EINVAL;
  return le::status(with_dtype(dtype, [&](auto t) {
    using T = decltype(t);
    le::rope_kernel<T><<<n_tokens, le::kThreads, 0, stream>>>(static_cast<T*>(x), positions, cos_table, sin_table,
                                                               heads, head_dim, row_stride, max_pos);
    return hipGetLastError();
  }));
}

}  // extern "C"
