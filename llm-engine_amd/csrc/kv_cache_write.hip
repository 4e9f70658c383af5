// K/V cache-write scatter (hot-path part 2).
//
// Reference: launch_store_kv / store_kv_kernel, src/kernels/store_kv.cu:20-36,
// and the CPU twin cpu_model.cpp:153-157:
//     k_cache[slots[t] * kv_dim + j] = k[t * kv_dim + j]   (v likewise)
//
// gfx950 design: HBM-bound byte movement, so every thread moves one 8-element
// chunk (32 B of fp32 or 16 B of bf16/fp16) of one row of K or V, consecutive
// threads take consecutive chunks of the same row, and the grid is sized to
// the row count rather than strided, so a 544-token step is a single wave of
// ~550 workgroups-worth of 16-byte transactions. K and V share the launch.
#include <type_traits>

#include "le_common.h"
#include "le_internal.h"

namespace le {
namespace {

// Copy-through when the types match keeps the bits without a round trip
// through float (exact anyway, but it costs VALU work).
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
  if constexpr (std::is_same_v<S, C>) {
    constexpr int n16 = sizeof(S) * 8 / 16;
#pragma unroll
    for (int i = 0; i < n16; i++)
      reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
  } else {
    float tmp[8];
    elem<S>::load8(src, tmp);
    elem<C>::store8(dst, tmp);
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

hipError_t kv_cache_write(const void* k, const void* v, int src_dtype, const int32_t* slots,
                          void* kc, void* vc, int cache_dtype, int n_tokens, int kv_dim,
                          int64_t num_slots, hipStream_t stream) {
  return with_dtype(src_dtype, [&](auto s) {
    return with_dtype(cache_dtype, [&](auto c) {
      return launch<decltype(s), decltype(c)>(k, v, slots, kc, vc, n_tokens, kv_dim, num_slots, stream);
    });
  });
}

}  // namespace le
