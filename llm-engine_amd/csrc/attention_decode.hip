// Paged decode attention with GQA-group sharing and split-K (hot-path parts
// 3, 4): the decode-row kernel. The workgroup itself (tiles, online softmax,
// in-launch merge of split rows) is decode_wg in attention_decode_wg.h, which
// the fused ragged kernel (attention_ragged.hip) shares.
#include "attention_decode_wg.h"

#include <atomic>

namespace le {
namespace {

constexpr int kMfmaWaves = 4;  // 8 waves measured slower (17.9 against 17.2 us)
constexpr int kMfmaThreads = kMfmaWaves * 64;

// Three instantiations of one workgroup body, by the registers they may use
// and the rows they take:
// * mfma_kernel: two waves per SIMD (two workgroups per CU, at most 256
//   registers a lane; 232 VGPRs, no spill). Launches of fewer than 512
//   workgroups run in one round. A TinyLlama-shaped decode step (64 rows of
//   128-1280 keys, 4 kv heads, 416 workgroups): 15.7 us per launch, against
//   19.8 in two rounds at one wave per SIMD.
// * mfma_kernel_wide: no bound (234 VGPRs plus 24 AGPRs as spill slots, one
//   wave per SIMD). For plans of 512 workgroups or more, two rounds of one
//   per CU (not fixed-layout plans, whose empty slots inflate the count):
//   the 64 x 4096 point (512 workgroups) 27.4 against 27.6 us at two per CU.
// * mfma_kernel_fold: rows straight from the stacked QKV projection with the
//   folded pre-attention norm (p.rms_x), at two per CU. The row scale's loads
//   issued ahead of the q and K/V row loads that use it: a TinyLlama-shaped
//   step 18.4 against 19.7 us with the scale formed before them.
template <typename ACT, typename KV, int HD>
__global__ __launch_bounds__(kMfmaThreads) __attribute__((amdgpu_waves_per_eu(2))) void mfma_kernel(DecodeParams p) {
  __shared__ dec::DecodeSmem<KV, HD, kMfmaWaves> sm;
  dec::decode_wg<ACT, KV, HD, kMfmaWaves>(p, sm, blockIdx.x, blockIdx.y, blockIdx.z);
}
template <typename ACT, typename KV, int HD>
__global__ __launch_bounds__(kMfmaThreads) __attribute__((amdgpu_waves_per_eu(2))) void mfma_kernel_fold(DecodeParams p) {
  __shared__ dec::DecodeSmem<KV, HD, kMfmaWaves> sm;
  dec::decode_wg<ACT, KV, HD, kMfmaWaves, true>(p, sm, blockIdx.x, blockIdx.y, blockIdx.z);
}
template <typename ACT, typename KV, int HD>
__global__ __launch_bounds__(kMfmaThreads) void mfma_kernel_wide(DecodeParams p) {
  __shared__ dec::DecodeSmem<KV, HD, kMfmaWaves> sm;
  dec::decode_wg<ACT, KV, HD, kMfmaWaves>(p, sm, blockIdx.x, blockIdx.y, blockIdx.z);
}

template <typename ACT, typename KV>
hipError_t launch(const DecodeParams& p, hipStream_t s) {
  const dim3 grid(p.n_rows, p.kv_heads, p.items ? 1 : p.nsplit);
  const bool wide = p.wide != 0;
  if (p.rms_x && p.rope_max_pos > 0) {
    if (p.head_dim == 64) mfma_kernel_fold<ACT, KV, 64><<<grid, kMfmaThreads, 0, s>>>(p);
    else mfma_kernel_fold<ACT, KV, 128><<<grid, kMfmaThreads, 0, s>>>(p);
  } else if (p.head_dim == 64) {
    if (wide) mfma_kernel_wide<ACT, KV, 64><<<grid, kMfmaThreads, 0, s>>>(p);
    else mfma_kernel<ACT, KV, 64><<<grid, kMfmaThreads, 0, s>>>(p);
  } else {
    if (wide) mfma_kernel_wide<ACT, KV, 128><<<grid, kMfmaThreads, 0, s>>>(p);
    else mfma_kernel<ACT, KV, 128><<<grid, kMfmaThreads, 0, s>>>(p);
  }
  return hipGetLastError();
}

}  // namespace


namespace {
__global__ void xcd_probe_kernel(int* out) {
  if (threadIdx.x == 0) {
    unsigned v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    out[blockIdx.x + blockIdx.y * gridDim.x] = static_cast<int>(v & 0xf);
  }
}

constexpr int kProbeW = 1000, kProbeH = 2;
__device__ int g_xcd_probe[kProbeW * kProbeH];  // static: the check allocates nothing
constexpr int kMaxDevices = 64;
std::atomic<int> g_placement[kMaxDevices];  // per device: 0 unknown, 1 holds, 2 does not

// 1-D and 2-D grids of the sizes the attention launches use, wider than the
// chip: ids equal modulo 8 must share an XCD, wherever the deal starts.
bool probe_placement(hipStream_t stream) {
  int* d = nullptr;
  if (hipGetSymbolAddress(reinterpret_cast<void**>(&d), HIP_SYMBOL(g_xcd_probe)) != hipSuccess) return false;
  static thread_local int h[kProbeW * kProbeH];
  bool ok = true;
  for (int shape = 0; shape < 2 && ok; shape++) {
    const dim3 grid = shape == 0 ? dim3(kProbeW * kProbeH) : dim3(kProbeW, kProbeH);
    xcd_probe_kernel<<<grid, 64, 0, stream>>>(d);
    ok = hipGetLastError() == hipSuccess &&
         hipMemcpyAsync(h, d, sizeof(h), hipMemcpyDeviceToHost, stream) == hipSuccess &&
         hipStreamSynchronize(stream) == hipSuccess;
    for (int i = 0; ok && i < kProbeW * kProbeH; i++) ok = h[i] == (h[0] + i) % 8;
  }
  return ok;
}
}  // namespace

bool xcd_placement_holds(hipStream_t stream) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  int st = g_placement[dev].load();
  if (st == 0) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
      return false;  // no probe inside a capture; the write-through stores are correct anywhere
    st = probe_placement(stream) ? 1 : 2;
    g_placement[dev].store(st);
  }
  return st == 1;
}

int decode_nsplit(int n_tokens, int kv_heads) {
  const int rows = n_tokens * kv_heads;
  const int target = 2048;  // 8 workgroups per CU on 256 CUs
  int ns = (target + rows - 1) / rows;
  return ns < 1 ? 1 : (ns > 32 ? 32 : ns);
}

hipError_t attention_decode(const DecodeParams& p, int act_dtype, int kv_dtype, hipStream_t s) {
  if (p.n_rows <= 0) return hipSuccess;
  return with_dtype(act_dtype, [&](auto a) {
    return with_dtype(kv_dtype, [&](auto k) { return launch<decltype(a), decltype(k)>(p, s); });
  });
}


}  // namespace le

#ifdef LE_TIMING
// Measurement builds only (build.py --timing): the decode workgroups' phase
// stamps of the last launch, [workgroup][8] uint64 (see g_timing).
extern "C" int le_timing_read(void* host, int64_t bytes) {
  return static_cast<int>(hipMemcpyFromSymbol(host, HIP_SYMBOL(le::g_timing), static_cast<size_t>(bytes), 0,
                                              hipMemcpyDeviceToHost));
}
#endif
