// K/V cache-write scatter (hot-path part 2).
//
// Reference: launch_store_kv / store_kv_kernel, src/kernels/store_kv.cu:20-36,
// and the CPU twin cpu_model.cpp:153-157:
//     k_cache[slots[t] * kv_dim + j] = k[t * kv_dim + j]   (v likewise)
//
// gfx950 design: HBM-bound byte movement, so every thread moves one 8-element
// chunk (32 B of fp32 or 16 B of bf16) of one row of K or V, consecutive
// threads take consecutive chunks of the same row, and the grid is sized to
// the row count rather than strided, so a 544-token step is a single wave of
// ~550 workgroups-worth of 16-byte transactions. K and V share the launch.
#include "le_common.h"
#include "le_internal.h"

namespace le {
namespace {

template <typename S> struct src_chunk;
template <> struct src_chunk<float> {
  __device__ __forceinline__ static void load(const float* p, float* o) {
    const uint4 a = ld16(p), b = ld16(p + 4);
    o[0] = __uint_as_float(a.x); o[1] = __uint_as_float(a.y);
    o[2] = __uint_as_float(a.z); o[3] = __uint_as_float(a.w);
    o[4] = __uint_as_float(b.x); o[5] = __uint_as_float(b.y);
    o[6] = __uint_as_float(b.z); o[7] = __uint_as_float(b.w);
  }
};
template <> struct src_chunk<bf16_t> {
  __device__ __forceinline__ static void load(const bf16_t* p, float* o) {
    elem<bf16_t>::widen(ld16(p), o);
  }
};

template <typename C> struct dst_chunk;
template <> struct dst_chunk<float> {
  __device__ __forceinline__ static void store(float* p, const float* v) {
    uint4 a, b;
    a.x = __float_as_uint(v[0]); a.y = __float_as_uint(v[1]);
    a.z = __float_as_uint(v[2]); a.w = __float_as_uint(v[3]);
    b.x = __float_as_uint(v[4]); b.y = __float_as_uint(v[5]);
    b.z = __float_as_uint(v[6]); b.w = __float_as_uint(v[7]);
    reinterpret_cast<uint4*>(p)[0] = a;
    reinterpret_cast<uint4*>(p)[1] = b;
  }
};
template <> struct dst_chunk<bf16_t> {
  __device__ __forceinline__ static void store(bf16_t* p, const float* v) {
    uint4 a;
    a.x = pack_bf16x2(v[0], v[1]); a.y = pack_bf16x2(v[2], v[3]);
    a.z = pack_bf16x2(v[4], v[5]); a.w = pack_bf16x2(v[6], v[7]);
    *reinterpret_cast<uint4*>(p) = a;
  }
};

// Copy-through when the types match keeps bf16 -> bf16 bit-exact without a
// round trip through float (which is exact anyway, but costs VALU).
template <typename S, typename C>
__global__ __launch_bounds__(256) void kv_cache_write_kernel(
    const S* __restrict__ k, const S* __restrict__ v, const int32_t* __restrict__ slots,
    C* __restrict__ k_cache, C* __restrict__ v_cache, int n_tokens, int kv_dim,
    int64_t num_slots) {
  const int chunks = kv_dim >> 3;
  const int64_t total = static_cast<int64_t>(n_tokens) * chunks * 2;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int t = static_cast<int>(idx / (2 * chunks));
  const int rem = static_cast<int>(idx - static_cast<int64_t>(t) * 2 * chunks);
  const int which = rem >= chunks;         // 0 = K, 1 = V
  const int c = rem - which * chunks;
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) return;
  const S* src = (which ? v : k) + static_cast<int64_t>(t) * kv_dim + c * 8;
  C* dst = (which ? v_cache : k_cache) + slot * kv_dim + c * 8;
  if constexpr (sizeof(S) == sizeof(C)) {
    constexpr int n16 = sizeof(S) * 8 / 16;
#pragma unroll
    for (int i = 0; i < n16; i++)
      reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
  } else {
    float tmp[8];
    src_chunk<S>::load(src, tmp);
    dst_chunk<C>::store(dst, tmp);
  }
}

template <typename S, typename C>
hipError_t launch(const void* k, const void* v, const int32_t* slots, void* kc, void* vc,
                  int n_tokens, int kv_dim, int64_t num_slots, hipStream_t stream) {
  const int64_t total = static_cast<int64_t>(n_tokens) * (kv_dim / 8) * 2;
  const int threads = 256;
  const int64_t blocks = (total + threads - 1) / threads;
  kv_cache_write_kernel<S, C><<<dim3(static_cast<unsigned>(blocks)), threads, 0, stream>>>(
      static_cast<const S*>(k), static_cast<const S*>(v), slots, static_cast<C*>(kc),
      static_cast<C*>(vc), n_tokens, kv_dim, num_slots);
  return hipGetLastError();
}

}  // namespace

hipError_t kv_cache_write(const void* k, const void* v, int src_bf16, const int32_t* slots,
                          void* kc, void* vc, int cache_bf16, int n_tokens, int kv_dim,
                          int64_t num_slots, hipStream_t stream) {
  if (src_bf16) {
    return cache_bf16 ? launch<bf16_t, bf16_t>(k, v, slots, kc, vc, n_tokens, kv_dim, num_slots, stream)
                      : launch<bf16_t, float>(k, v, slots, kc, vc, n_tokens, kv_dim, num_slots, stream);
  }
  return cache_bf16 ? launch<float, bf16_t>(k, v, slots, kc, vc, n_tokens, kv_dim, num_slots, stream)
                    : launch<float, float>(k, v, slots, kc, vc, n_tokens, kv_dim, num_slots, stream);
}

}  // namespace le
