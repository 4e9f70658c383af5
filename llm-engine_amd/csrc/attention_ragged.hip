// Ragged paged attention of a mixed step in one launch (hot-path part 3):
// the step's prefill-chunk rows (chunk_wg, attention_chunk_wg.h) and decode
// rows (decode_wg, attention_decode_wg.h) as workgroups of one grid.
//
// With two launches the chunk rows' latency-bound phases (stage, compute,
// partial store, merge) and the decode rows' HBM streaming run one after the
// other, with a launch gap between them. In one grid the decode workgroups
// stream on the CUs the chunk workgroups leave free, and start on the others
// as chunk workgroups retire. Chunk workgroups come first in the grid: theirs
// is the longer dependent chain (a split tile's merge waits for its last
// partition).
//
// Both kinds keep their own merges inside the launch: partition indices and
// arrival counters are disjoint between them (the plan numbers partitions
// across both lists; counters are indexed by a row's or tile's first token).
// Workgroups are 512 threads (the chunk workgroup's eight waves); the decode
// workgroups run as eight waves as well. The LDS is the larger of the two.
#include "attention_chunk_wg.h"
#include "attention_decode_wg.h"

namespace le {
namespace {

constexpr int kRaggedThreads = chk::kThreads;
constexpr int kDecodeWaves = kRaggedThreads / kWave;

template <typename KV, int HD> union RaggedSmem {
  chk::ChunkSmem<KV, HD> c;
  dec::DecodeSmem<KV, HD, kDecodeWaves> d;
};

template <typename ACT, typename KV, int HD>
__global__ __launch_bounds__(kRaggedThreads) void ragged_kernel(DecodeParams dp, ChunkParams cp) {
  __shared__ RaggedSmem<KV, HD> sm;
  const int n_chunk_wg = cp.n_items * cp.kv_heads;
  const int b = blockIdx.x;
  if (b < n_chunk_wg) {
    // item-major within each kv head, as the chunk kernel's 2-D grid (the
    // plan places a split tile's partitions at item indices equal modulo 8)
    chk::chunk_wg<ACT, KV, HD>(cp, sm.c, b % cp.n_items, b / cp.n_items);
  } else {
    // item-major within each kv head, as the decode kernel's 2-D grid: the
    // plan places a split row's partitions at item indices equal modulo 8,
    // so they share an XCD in either launch
    const int d = b - n_chunk_wg;
    dec::decode_wg<ACT, KV, HD, kDecodeWaves>(dp, sm.d, d % dp.n_rows, d / dp.n_rows, 0);
  }
}

}  // namespace


hipError_t attention_ragged(const DecodeParams& d, const ChunkParams& c, int act_dtype, int kv_dtype,
                            hipStream_t s) {
  const int64_t n = static_cast<int64_t>(c.n_items + d.n_rows) * c.kv_heads;
  if (n <= 0) return hipSuccess;
  if (n > 0x7fffffff || d.kv_heads != c.kv_heads || d.head_dim != c.head_dim || !d.items)
    return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(n));
  return with_dtype(act_dtype, [&](auto a) {
    return with_dtype(kv_dtype, [&](auto k) {
      using ACT = decltype(a);
      using KV = decltype(k);
      if (c.head_dim == 64) ragged_kernel<ACT, KV, 64><<<grid, kRaggedThreads, 0, s>>>(d, c);
      else ragged_kernel<ACT, KV, 128><<<grid, kRaggedThreads, 0, s>>>(d, c);
      return hipGetLastError();
    });
  });
}

}  // namespace le

#ifdef LE_TIMING
// Measurement builds only: the mixed-step kernel's phase stamps of its last
// launch (decode and chunk workgroups; slot 7 tells them apart).
extern "C" int le_timing_read_ragged(void* host, int64_t bytes) {
  return static_cast<int>(hipMemcpyFromSymbol(host, HIP_SYMBOL(le::g_timing), static_cast<size_t>(bytes), 0,
                                              hipMemcpyDeviceToHost));
}
#endif
