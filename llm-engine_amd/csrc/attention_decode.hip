// Paged decode attention with GQA-group sharing and split-K (hot-path parts
// 3, 4): the decode-row kernel. The workgroup itself (tiles, online softmax,
// in-launch merge of split rows) is decode_wg in attention_decode_wg.h, which
// the fused ragged kernel (attention_ragged.hip) shares.
#include "attention_decode_wg.h"

namespace le {
namespace {

#ifndef LE_DECODE_WAVES
#define LE_DECODE_WAVES 4
#endif
constexpr int kMfmaWaves = LE_DECODE_WAVES;
constexpr int kMfmaThreads = kMfmaWaves * 64;

template <typename ACT, typename KV, int HD>
__global__ __launch_bounds__(kMfmaThreads) void mfma_kernel(DecodeParams p) {
  __shared__ dec::DecodeSmem<KV, HD, kMfmaWaves> sm;
  dec::decode_wg<ACT, KV, HD, kMfmaWaves>(p, sm, blockIdx.x, blockIdx.y, blockIdx.z);
}

template <typename ACT>
hipError_t dispatch(const DecodeParams& p, int kv_bf16, hipStream_t s) {
  const dim3 grid(p.n_rows, p.kv_heads, p.items ? 1 : p.nsplit);
  if (kv_bf16) {
    if (p.head_dim == 64) mfma_kernel<ACT, bf16_t, 64><<<grid, kMfmaThreads, 0, s>>>(p);
    else mfma_kernel<ACT, bf16_t, 128><<<grid, kMfmaThreads, 0, s>>>(p);
    return hipGetLastError();
  }
  if (p.head_dim == 64) mfma_kernel<ACT, float, 64><<<grid, kMfmaThreads, 0, s>>>(p);
  else mfma_kernel<ACT, float, 128><<<grid, kMfmaThreads, 0, s>>>(p);
  return hipGetLastError();
}


}  // namespace

#ifdef LE_PROBE_TIMING
extern "C" int le_probe_timing(void* host, size_t bytes) {
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(dec::g_probe_ts), bytes < sizeof(dec::g_probe_ts) ? bytes : sizeof(dec::g_probe_ts)) == hipSuccess ? 0 : 1;
}
extern "C" int le_probe_timing_clear(void) {
  static uint64_t zeros[16384][8];
  return hipMemcpyToSymbol(HIP_SYMBOL(dec::g_probe_ts), zeros, sizeof(zeros)) == hipSuccess ? 0 : 1;
}
#endif

int decode_nsplit(int n_tokens, int kv_heads) {
  const int rows = n_tokens * kv_heads;
  const int target = 2048;  // 8 workgroups per CU on 256 CUs
  int ns = (target + rows - 1) / rows;
  return ns < 1 ? 1 : (ns > 32 ? 32 : ns);
}

hipError_t attention_decode(const DecodeParams& p, int act_bf16, int kv_bf16, hipStream_t s) {
  if (p.n_rows <= 0) return hipSuccess;
  return act_bf16 ? dispatch<bf16_t>(p, kv_bf16, s) : dispatch<float>(p, kv_bf16, s);
}


}  // namespace le
