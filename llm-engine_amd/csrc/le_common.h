// Device helpers shared by the gfx950 kernels: bf16 conversion, 16-byte vector
// loads and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace le {

constexpr int kWave = 64;

// bf16 is carried as its raw 16-bit pattern: the cache, the activations and the
// MFMA operands all move it as bits, and widening is a shift.
struct bf16_t {
  uint16_t bits;
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round to nearest even, inf/nan passed through unrounded: the same rule as the
// host conversion the caches are checked against, so a stored bf16 is
// bit-identical to a host-rounded one.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u) return u >> 16;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

// Element type traits: VEC = elements per 16-byte load.
template <typename T> struct elem;
template <> struct elem<float> {
  static constexpr int VEC = 4;
  __device__ __forceinline__ static void widen(const uint4& r, float* o) {
    o[0] = __uint_as_float(r.x); o[1] = __uint_as_float(r.y);
    o[2] = __uint_as_float(r.z); o[3] = __uint_as_float(r.w);
  }
  __device__ __forceinline__ static float load1(const float* p) { return *p; }
  __device__ __forceinline__ static void store1(float* p, float v) { *p = v; }
};
template <> struct elem<bf16_t> {
  static constexpr int VEC = 8;
  __device__ __forceinline__ static void widen(const uint4& r, float* o) {
    o[0] = bf16_lo(r.x); o[1] = bf16_hi(r.x); o[2] = bf16_lo(r.y); o[3] = bf16_hi(r.y);
    o[4] = bf16_lo(r.z); o[5] = bf16_hi(r.z); o[6] = bf16_lo(r.w); o[7] = bf16_hi(r.w);
  }
  __device__ __forceinline__ static float load1(const bf16_t* p) {
    return __uint_as_float(static_cast<uint32_t>(p->bits) << 16);
  }
  __device__ __forceinline__ static void store1(bf16_t* p, float v) {
    p->bits = static_cast<uint16_t>(f32_to_bf16_bits(v));
  }
};

__device__ __forceinline__ uint4 ld16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}
// K/V history load (read once per step). A non-temporal variant measured no
// faster on the decode rows.
__device__ __forceinline__ uint4 ld16_stream(const void* p) { return ld16(p); }

// Cross-lane moves inside a 16-lane DPP row: no LDS traffic, one VALU op each.
namespace dpp {
constexpr int kXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kHalfMirror = 0x141; // lane i <-> 7-i within each 8 lanes
constexpr int kMirror = 0x140;     // lane i <-> 15-i within each 16 lanes
template <int CTRL>
__device__ __forceinline__ float mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
}  // namespace dpp

// Sum over groups of N adjacent lanes (N a power of two <= 64); every lane of
// the group ends with the group's total. Steps inside a 16-lane row are DPP;
// the pairing is a permutation, not a shift, so after steps 1..k every lane of
// a 2^k group holds that group's sum and the next step pairs it with the
// neighbouring group.
template <int N>
__device__ __forceinline__ float group_sum(float v) {
  if (N >= 2) v += dpp::mov<dpp::kXor1>(v);
  if (N >= 4) v += dpp::mov<dpp::kXor2>(v);
  if (N >= 8) v += dpp::mov<dpp::kHalfMirror>(v);
  if (N >= 16) v += dpp::mov<dpp::kMirror>(v);
  if (N >= 32) v += __shfl_xor(v, 16, kWave);
  if (N >= 64) v += __shfl_xor(v, 32, kWave);
  return v;
}

template <int N>
__device__ __forceinline__ float group_max(float v) {
  if (N >= 2) v = fmaxf(v, dpp::mov<dpp::kXor1>(v));
  if (N >= 4) v = fmaxf(v, dpp::mov<dpp::kXor2>(v));
  if (N >= 8) v = fmaxf(v, dpp::mov<dpp::kHalfMirror>(v));
  if (N >= 16) v = fmaxf(v, dpp::mov<dpp::kMirror>(v));
  if (N >= 32) v = fmaxf(v, __shfl_xor(v, 16, kWave));
  if (N >= 64) v = fmaxf(v, __shfl_xor(v, 32, kWave));
  return v;
}

// Whole-wave reductions: DPP inside each 16-lane row, then the four row
// results are read as scalars. The result is wave-uniform.
__device__ __forceinline__ float wave_max(float v) {
  v = group_max<16>(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

__device__ __forceinline__ float wave_sum(float v) {
  v = group_sum<16>(v);
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

// Device-coherent 16-byte accesses for data exchanged between workgroups
// (possibly on different XCDs, whose L2s are not coherent with each other):
// raw buffer loads/stores with the sc1 cache-policy bit, the same policy the
// compiler gives agent-scope relaxed atomics, so a reader never hits a stale
// line left in its own L2. The compiler tracks these loads like any other.
typedef float f32x4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coherent_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7FFFFFFF, 0x00020000);
}
constexpr int kCachePolicySc1 = 16;
typedef uint32_t u32x4raw __attribute__((vector_size(16)));  // the builtins' data type
__device__ __forceinline__ f32x4v ld_coherent16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  const u32x4raw v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kCachePolicySc1);
  return __builtin_bit_cast(f32x4v, v);
}
__device__ __forceinline__ void st_coherent16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, f32x4v v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4raw, v), r, byte_off, 0, kCachePolicySc1);
}
// A plain 16-byte store (write-back into the XCD's L2), for data that only
// workgroups on the same XCD read back.
__device__ __forceinline__ void st_l2_16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, f32x4v v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4raw, v), r, byte_off, 0, 0);
}
typedef uint32_t u32x2raw __attribute__((vector_size(8)));
__device__ __forceinline__ void st_coherent8(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, uint2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2raw, v), r, byte_off, 0, kCachePolicySc1);
}
__device__ __forceinline__ uint4 ld_coherent16u(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  const u32x4raw v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kCachePolicySc1);
  return __builtin_bit_cast(uint4, v);
}

}  // namespace le
