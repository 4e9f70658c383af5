// Chunked-prefill attention on MFMA (hot-path part 3, prefill-chunk rows):
// the chunk-row kernel. The workgroup itself is chunk_wg in
// attention_chunk_wg.h, which the fused ragged kernel (attention_ragged.hip)
// shares.
#include "attention_chunk_wg.h"

namespace le {
namespace {

template <typename ACT, int HD>
__global__ __launch_bounds__(chk::kThreads) void chunk_kernel(ChunkParams p) {
  __shared__ chk::ChunkSmem<HD> sm;
  chk::chunk_wg<ACT, HD>(p, sm, blockIdx.x, blockIdx.y);
}

}  // namespace


hipError_t attention_chunk(const ChunkParams& p, int act_bf16, hipStream_t s) {
  if (p.n_items <= 0) return hipSuccess;
  const dim3 grid(p.n_items, p.kv_heads);
  if (p.head_dim == 64) {
    if (act_bf16) chunk_kernel<bf16_t, 64><<<grid, chk::kThreads, 0, s>>>(p);
    else chunk_kernel<float, 64><<<grid, chk::kThreads, 0, s>>>(p);
  } else {
    if (act_bf16) chunk_kernel<bf16_t, 128><<<grid, chk::kThreads, 0, s>>>(p);
    else chunk_kernel<float, 128><<<grid, chk::kThreads, 0, s>>>(p);
  }
  return hipGetLastError();
}

}  // namespace le
