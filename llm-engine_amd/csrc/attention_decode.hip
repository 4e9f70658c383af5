// Paged decode attention with GQA-group sharing and split-K (hot-path parts
// 3, 4): the decode-row kernel. The workgroup itself (tiles, online softmax,
// in-launch merge of split rows) is decode_wg in attention_decode_wg.h, which
// the fused ragged kernel (attention_ragged.hip) shares.
#include "attention_decode_wg.h"

namespace le {
namespace {

constexpr int kMfmaWaves = 4;  // 8 waves measured slower (17.9 against 17.2 us)
constexpr int kMfmaThreads = kMfmaWaves * 64;

template <typename ACT, typename KV, int HD>
__global__ __launch_bounds__(kMfmaThreads) void mfma_kernel(DecodeParams p) {
  __shared__ dec::DecodeSmem<KV, HD, kMfmaWaves> sm;
  dec::decode_wg<ACT, KV, HD, kMfmaWaves>(p, sm, blockIdx.x, blockIdx.y, blockIdx.z);
}

template <typename ACT, typename KV>
hipError_t launch(const DecodeParams& p, hipStream_t s) {
  const dim3 grid(p.n_rows, p.kv_heads, p.items ? 1 : p.nsplit);
  if (p.head_dim == 64) mfma_kernel<ACT, KV, 64><<<grid, kMfmaThreads, 0, s>>>(p);
  else mfma_kernel<ACT, KV, 128><<<grid, kMfmaThreads, 0, s>>>(p);
  return hipGetLastError();
}

}  // namespace


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
  return static_cast<int>(hipMemcpyFromSymbol(host, HIP_SYMBOL(le::dec::g_timing), static_cast<size_t>(bytes), 0,
                                              hipMemcpyDeviceToHost));
}
#endif
