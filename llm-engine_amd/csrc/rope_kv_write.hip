// Bias + RoPE + K/V cache-write scatter in one launch (hot-path part 2, fused
// with what produces its rows).
//
// Reference: the per-layer sequence cuda_model.cu:358-368 -- launch_add_bias on
// q, k, v (elementwise.cu:40), launch_rope on q and k (rope.cu:53, rotate_half
// as in ops.h:55-66), launch_store_kv (store_kv.cu:20-36) -- six launches and
// three round trips of the q/k/v rows through HBM. Here the fused QKV
// projection output is read once: each workgroup takes one token, applies the
// bias, rotates q and k with the token's position, writes q contiguously for
// attention and scatters k and v straight into the paged caches at the
// token's slot.
//
// Work unit per thread: four rotation pairs (i..i+3 with i+half..i+half+3) of
// one q or k head, or eight elements of v, so every global access is an 8- or
// 16-byte vector and the cos/sin rows are read as float4.
#include "le_common.h"
#include "le_internal.h"

namespace le {
namespace {

// No contraction: a*c - b*s is two roundings of products and one of the
// difference, as the reference's CPU op computes it.
#pragma clang fp contract(off)

template <typename T, typename C>
__global__ __launch_bounds__(256) void rope_kv_write_kernel(
    const T* __restrict__ qkv, int64_t stride, const float* __restrict__ bias,
    const int32_t* __restrict__ positions, const int32_t* __restrict__ slots,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, int max_pos, int nh, int nkv,
    int hd, T* __restrict__ q_out, C* __restrict__ kc, C* __restrict__ vc, int64_t num_slots,
    const T* __restrict__ rms_x, int rms_hidden, float rms_eps) {
  const int t = blockIdx.x;
  // the folded pre-attention RMSNorm: every wave forms the row's scale
  const bool scaled = rms_x != nullptr;
  const float rs = scaled ? row_rms_scale(rms_x + static_cast<int64_t>(t) * rms_hidden, rms_hidden, rms_eps) : 1.f;
  const int pos = positions[t];
  const bool pos_ok = pos >= 0 && pos < max_pos;
  const int64_t slot = slots[t];
  const bool kv_ok = pos_ok && slot >= 0 && slot < num_slots;
  const int half = hd >> 1, qd = nh * hd, kvd = nkv * hd;
  const int gph = half >> 2;  // 4-pair groups per head
  const int n_rope = (nh + nkv) * gph;
  const int n_units = n_rope + (kvd >> 3);
  const T* row = qkv + static_cast<int64_t>(t) * stride;
  const int64_t tab = static_cast<int64_t>(pos_ok ? pos : 0) * half;
  for (int u = threadIdx.x; u < n_units; u += blockDim.x) {
    if (u < n_rope) {
      const int h = u / gph;
      const int i = (u - h * gph) * 4;
      const int off = h * hd + i;
      float a[4], b[4];
      elem<T>::load4(row + off, a);
      elem<T>::load4(row + off + half, b);
      if (scaled) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
          a[e] = elem<T>::round(bias ? a[e] * rs + bias[off + e] : a[e] * rs);
          b[e] = elem<T>::round(bias ? b[e] * rs + bias[off + half + e] : b[e] * rs);
        }
      } else if (bias) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
          a[e] = elem<T>::round(a[e] + bias[off + e]);
          b[e] = elem<T>::round(b[e] + bias[off + half + e]);
        }
      }
      float ra[4], rb[4];
      const float4 c4 = *reinterpret_cast<const float4*>(cos_t + tab + i);
      const float4 s4 = *reinterpret_cast<const float4*>(sin_t + tab + i);
      const float c[4] = {c4.x, c4.y, c4.z, c4.w}, s[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
      for (int e = 0; e < 4; e++) {
        ra[e] = pos_ok ? a[e] * c[e] - b[e] * s[e] : 0.f;
        rb[e] = pos_ok ? b[e] * c[e] + a[e] * s[e] : 0.f;
      }
      if (h < nh) {
        T* dst = q_out + static_cast<int64_t>(t) * qd + off;
        elem<T>::store4(dst, ra);
        elem<T>::store4(dst + half, rb);
      } else if (kv_ok) {
        C* dst = kc + slot * kvd + (off - qd);
        elem<C>::store4(dst, ra);
        elem<C>::store4(dst + half, rb);
      }
    } else if (kv_ok) {
      const int j = (u - n_rope) * 8;
      float x[8];
      elem<T>::load4(row + qd + kvd + j, x);
      elem<T>::load4(row + qd + kvd + j + 4, x + 4);
      if (scaled) {
#pragma unroll
        for (int e = 0; e < 8; e++) x[e] = elem<T>::round(bias ? x[e] * rs + bias[qd + kvd + j + e] : x[e] * rs);
      } else if (bias) {
#pragma unroll
        for (int e = 0; e < 8; e++) x[e] = elem<T>::round(x[e] + bias[qd + kvd + j + e]);
      }
      C* dst = vc + slot * kvd + j;
      elem<C>::store4(dst, x);
      elem<C>::store4(dst + 4, x + 4);
    }
  }
}

template <typename T, typename C>
hipError_t launch(const void* qkv, int64_t stride, const float* bias, const int32_t* positions,
                  const int32_t* slots, const float* cos_t, const float* sin_t, int max_pos, int n,
                  int nh, int nkv, int hd, void* q_out, void* kc, void* vc, int64_t num_slots,
                  const void* rms_x, int rms_hidden, float rms_eps, hipStream_t stream) {
  rope_kv_write_kernel<T, C><<<dim3(static_cast<unsigned>(n)), 256, 0, stream>>>(
      static_cast<const T*>(qkv), stride, bias, positions, slots, cos_t, sin_t, max_pos, nh, nkv, hd,
      static_cast<T*>(q_out), static_cast<C*>(kc), static_cast<C*>(vc), num_slots, static_cast<const T*>(rms_x),
      rms_hidden, rms_eps);
  return hipGetLastError();
}

}  // namespace

hipError_t rope_kv_cache_write(const void* qkv, int act_dtype, int64_t row_stride, const float* bias,
                               const int32_t* positions, const int32_t* slots, const float* cos_t,
                               const float* sin_t, int max_pos, int n_tokens, int q_heads,
                               int kv_heads, int head_dim, void* q_out, void* kc, void* vc,
                               int cache_dtype, int64_t num_slots, hipStream_t stream, const void* rms_x,
                               int rms_hidden, float rms_eps) {
  return with_dtype(act_dtype, [&](auto a) {
    return with_dtype(cache_dtype, [&](auto c) {
      return launch<decltype(a), decltype(c)>(qkv, row_stride, bias, positions, slots, cos_t, sin_t, max_pos,
                                              n_tokens, q_heads, kv_heads, head_dim, q_out, kc, vc, num_slots,
                                              rms_x, rms_hidden, rms_eps, stream);
    });
  });
}

}  // namespace le
