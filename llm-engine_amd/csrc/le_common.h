// Device helpers shared by the gfx950 kernels: bf16/fp16 conversion, 16-byte vector
// loads and wave64 reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace le {

constexpr int kWave = 64;

// bf16 and fp16 are carried as raw 16-bit patterns: the caches, the
// activations and the MFMA operands all move them as bits.
struct bf16_t {
  uint16_t bits;
};
struct f16_t {
  uint16_t bits;
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round to nearest even, inf/nan passed through unrounded: the same rule as the
// host conversion the caches are checked against (tensor.h:23-28), so a
// stored bf16 is bit-identical to a host-rounded one.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u) return u >> 16;
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

// fp16: the hardware conversion rounds to nearest even, with subnormal
// results and overflow to infinity, as the host rule (tensor.h:38-56) does.
// A NaN becomes the host rule's quiet NaN (sign kept, payload 0x200).
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) & 0x8000u) | 0x7e00u;
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h & 0xffffu)));
}
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  return f32_to_f16_bits(lo) | (f32_to_f16_bits(hi) << 16);
}
__device__ __forceinline__ float f16_lo(uint32_t w) { return f16_bits_to_f32(w); }
__device__ __forceinline__ float f16_hi(uint32_t w) { return f16_bits_to_f32(w >> 16); }

__device__ __forceinline__ uint4 ld16(const void* p) {
  return *reinterpret_cast<const uint4*>(p);
}

// Element type traits. VEC = elements per 16-byte load; widen turns those 16
// bytes into floats; load/store move 4 or 8 consecutive elements as floats
// (stores round to the type); round(x) is x as the type would store it.
template <typename T> struct elem;
template <> struct elem<float> {
  static constexpr int VEC = 4;
  __device__ __forceinline__ static void widen(const uint4& r, float* o) {
    o[0] = __uint_as_float(r.x); o[1] = __uint_as_float(r.y);
    o[2] = __uint_as_float(r.z); o[3] = __uint_as_float(r.w);
  }
  __device__ __forceinline__ static float load1(const float* p) { return *p; }
  __device__ __forceinline__ static void store1(float* p, float v) { *p = v; }
  __device__ __forceinline__ static float round(float x) { return x; }
  __device__ __forceinline__ static void load4(const float* p, float* o) { widen(ld16(p), o); }
  __device__ __forceinline__ static void load8(const float* p, float* o) {
    widen(ld16(p), o);
    widen(ld16(p + 4), o + 4);
  }
  __device__ __forceinline__ static void store4(float* p, const float* v) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  }
  __device__ __forceinline__ static void store8(float* p, const float* v) {
    store4(p, v);
    store4(p + 4, v + 4);
  }
};

// The two 16-bit types share everything but the conversions.
template <typename T, float (*LO)(uint32_t), float (*HI)(uint32_t), uint32_t (*TO)(float),
          uint32_t (*PACK)(float, float)>
struct elem16 {
  static constexpr int VEC = 8;
  __device__ __forceinline__ static void widen(const uint4& r, float* o) {
    o[0] = LO(r.x); o[1] = HI(r.x); o[2] = LO(r.y); o[3] = HI(r.y);
    o[4] = LO(r.z); o[5] = HI(r.z); o[6] = LO(r.w); o[7] = HI(r.w);
  }
  __device__ __forceinline__ static float load1(const T* p) { return LO(p->bits); }
  __device__ __forceinline__ static void store1(T* p, float v) { p->bits = static_cast<uint16_t>(TO(v)); }
  __device__ __forceinline__ static float round(float x) { return LO(TO(x)); }
  __device__ __forceinline__ static void load4(const T* p, float* o) {
    const uint2 r = *reinterpret_cast<const uint2*>(p);
    o[0] = LO(r.x); o[1] = HI(r.x); o[2] = LO(r.y); o[3] = HI(r.y);
  }
  __device__ __forceinline__ static void load8(const T* p, float* o) { widen(ld16(p), o); }
  __device__ __forceinline__ static void store4(T* p, const float* v) {
    *reinterpret_cast<uint2*>(p) = make_uint2(PACK(v[0], v[1]), PACK(v[2], v[3]));
  }
  __device__ __forceinline__ static void store8(T* p, const float* v) {
    *reinterpret_cast<uint4*>(p) =
        make_uint4(PACK(v[0], v[1]), PACK(v[2], v[3]), PACK(v[4], v[5]), PACK(v[6], v[7]));
  }
};
template <> struct elem<bf16_t> : elem16<bf16_t, bf16_lo, bf16_hi, f32_to_bf16_bits, pack_bf16x2> {};
template <> struct elem<f16_t> : elem16<f16_t, f16_lo, f16_hi, f32_to_f16_bits, pack_f16x2> {};

// The 16-bit MFMA operand types and the 16x16x32 MFMA of each 16-bit type.
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
template <typename T> struct mma16;
template <> struct mma16<bf16_t> {
  using scalar = __bf16;
  using v8 = bf16x8;
  using v4 = bf16x4;
  __device__ __forceinline__ static f32x4 mma(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct mma16<f16_t> {
  using scalar = _Float16;
  using v8 = f16x8;
  using v4 = f16x4;
  __device__ __forceinline__ static f32x4 mma(v8 a, v8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// ds_read_b64_tr_b16: in each group of 16 lanes, lane i receives 16-bit
// element (i % 4) of the 8-byte chunks addressed by lanes 4j + i/4, j = 0..3.
template <typename T>
__device__ __forceinline__ typename mma16<T>::v4 lds_read_tr16(const char* p) {
  // C-style cast: the generic LDS pointer becomes an address-space-3 pointer.
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) i16x4*)(p));
  return __builtin_bit_cast(typename mma16<T>::v4, v);
}

// K/V history load (read once per step). A non-temporal variant measured no
// faster on the decode rows.
__device__ __forceinline__ uint4 ld16_stream(const void* p) { return ld16(p); }
__device__ __forceinline__ float4 as_float4(uint4 u) {
  return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
}

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

// Max / sum over the four 16-lane rows of a wave (lanes i, i^16, i^32 and
// i^48), every lane ending with the result. gfx950's row swaps
// (v_permlane32_swap, v_permlane16_swap: the two halves, then the odd and
// even rows, of two registers exchanged) are VALU moves; a shuffle through
// ds_bpermute is an LDS round trip that the wave waits for.
__device__ __forceinline__ float vmax2(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float rows_max(float v) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = vmax2(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return vmax2(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float rows_sum(float v) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
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

// 1/sqrt(mean(x^2) + eps) of one row of the residual stream (the folded
// pre-attention RMSNorm), formed by one wave alone: each lane sums the
// squares of its 16-byte pieces, then the wave reduces (no LDS, no barrier).
// Every wave that calls it on a row gets the same value (the decode kernel
// and rope_kv_write_kernel both use it).
template <typename ACT>
__device__ __forceinline__ float row_rms_scale(const ACT* x, int hidden, float eps) {
  constexpr int V = 16 / static_cast<int>(sizeof(ACT));
  const int lane = threadIdx.x & (kWave - 1);
  float ss = 0.f;
  for (int pc = lane; pc * V < hidden; pc += kWave) {
    float v[8];
    if constexpr (V == 8) {
      elem<ACT>::load8(x + pc * V, v);
    } else {
      elem<ACT>::load4(x + pc * V, v);
    }
#pragma unroll
    for (int e = 0; e < V; e++) ss += v[e] * v[e];
  }
  ss = wave_sum(ss);
  return 1.0f / sqrtf(ss / hidden + eps);
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
// Arrival counters of split rows: one per (row, kv head), zero between
// launches (the last arriver resets it).
typedef unsigned long long arrival_t;

// Plain stores (write-back into the XCD's L2), for partials that only
// workgroups on the same XCD read back (LE_PLAN_XCD_LOCAL).
__device__ __forceinline__ void st_l2_16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, f32x4v v) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4raw, v), r, byte_off, 0, 0);
}
typedef uint32_t u32x2raw __attribute__((vector_size(8)));
__device__ __forceinline__ void st_l2_8(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, uint2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2raw, v), r, byte_off, 0, 0);
}
__device__ __forceinline__ void st_coherent8(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, uint2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2raw, v), r, byte_off, 0, kCachePolicySc1);
}
__device__ __forceinline__ uint4 ld_coherent16u(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  const u32x4raw v = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, kCachePolicySc1);
  return __builtin_bit_cast(uint4, v);
}

// Calls f with a value of the element type a dtype code names (0 fp32,
// 1 bf16, 2 fp16), so host code picks a kernel instantiation in one place.
template <typename F>
__host__ __device__ inline auto with_dtype(int dt, F&& f) {
  if (dt == 1) return f(bf16_t{});
  if (dt == 2) return f(f16_t{});
  return f(float{});
}
// The same over the 16-bit types only (the MFMA kernels' operand types).
template <typename F>
__host__ __device__ inline auto with_dtype16(int dt, F&& f) {
  if (dt == 2) return f(f16_t{});
  return f(bf16_t{});
}

namespace {
// Phase stamps (measurement builds, -DLE_TIMING; no code otherwise): thread
// 0 of each attention workgroup records realtime stamps (100 MHz) of its phases
// and the CU/XCD it ran on, per linear workgroup id; the last launch's values
// stay. Slots: 0 start, 1 item and block ids staged, 2 tiles done, 3 output
// or partial written, 4 end (after the split row's arrival and merge),
// 5 HW_ID | XCC_ID << 32, 6 partition blocks << 32 | partitions of its row
// (or tile), 7 kind (1 decode, 2 chunk, 3 decode in a round-trip probe
// build, whose slots 8 and 9 hold the probe's stamps), 8 + w wave w's tiles
// done (chunk workgroups and the mixed-step kernel's decode workgroups; slot
// 2 is wave 0's). Chunk workgroups stamp 1 after their first
// stage is in LDS and 2 after their last tile.
#ifdef LE_TIMING
constexpr int kTimSlots = 16;
constexpr int kTimWorkgroups = 65536;
__device__ uint64_t g_timing[kTimWorkgroups * kTimSlots];
__device__ __forceinline__ void tim_put(int slot, uint64_t v) {
  if (threadIdx.x == 0) {
    const int64_t wg = blockIdx.x + static_cast<int64_t>(blockIdx.y) * gridDim.x;
    if (wg < kTimWorkgroups) g_timing[wg * kTimSlots + slot] = v;
  }
}
__device__ __forceinline__ void tim_put_wave(int slot, uint64_t v) {
  if ((threadIdx.x & 63) == 0) {
    const int64_t wg = blockIdx.x + static_cast<int64_t>(blockIdx.y) * gridDim.x;
    if (wg < kTimWorkgroups) g_timing[wg * kTimSlots + slot + (threadIdx.x >> 6)] = v;
  }
}
__device__ __forceinline__ uint64_t tim_place() {
  uint32_t hw, xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  return (static_cast<uint64_t>(xcc) << 32) | hw;
}
#define LE_TIM(slot, v) tim_put(slot, v)
#define LE_TIM_WAVE(slot, v) tim_put_wave(slot, v)
#define LE_TIM_NOW() __builtin_amdgcn_s_memrealtime()
#define LE_TIM_PLACE() tim_place()
#else
#define LE_TIM(slot, v) ((void)0)
#define LE_TIM_WAVE(slot, v) ((void)0)
#define LE_TIM_NOW() uint64_t{0}
#define LE_TIM_PLACE() uint64_t{0}
#endif

}  // namespace
}  // namespace le
