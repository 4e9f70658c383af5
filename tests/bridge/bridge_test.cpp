// Compiled C++ test of the drop-in boundary: calls the reference's launcher
// signatures (include/le_cuda_kernels.h = cuda_kernels.h:43-64) with fp16
// buffers on the GPU, the way cuda_model.cu:366-377 calls them for a decode
// step, and checks the results against the CPU oracle (oracle/oracle.c,
// ops.h:87-111) on the same fp16 values widened to fp32.
//
//   bridge_test [n_seqs] [seed]     exit 0 = pass; prints one summary line
//
// Case (config 2's shape): Qwen2.5-0.5B GQA (14 q heads, 2 kv heads,
// head_dim 64), block 16, contexts log-uniform in [64, 4096], block tables
// from a random permutation of a 32768-block pool. Each sequence's newest
// K/V row is scattered by launch_store_kv first; then both attention
// launchers run over the same step.
//   * caches: bit-identical to the oracle's scatter of the same rows;
//   * attention: max-abs error against the oracle below 6e-4 (the fp16
//     kernels' error on this shape is about 3e-4) plus the fp16 rounding of
//     the output (2^-11 relative, |out| < 4);
//   * launch_attention_decode and launch_attention_decode_gqa agree bit for
//     bit (the reference requires equal greedy tokens from its two kernels,
//     test_cuda_invariance.cpp:295-344);
//   * a rejected shape (head_dim 96) throws std::runtime_error, as the
//     reference's launchers do (attention_decode_gqa.cu:211-224).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <stdexcept>
#include <vector>

#include "le_cuda_kernels.h"
#include "llm_engine_amd.h"
#include "oracle.h"

namespace {

#define HIP_OK(x)                                                                   \
  do {                                                                              \
    hipError_t e_ = (x);                                                            \
    if (e_ != hipSuccess) {                                                         \
      std::fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));           \
      std::exit(2);                                                                 \
    }                                                                               \
  } while (0)

template <typename T>
T* to_device(const std::vector<T>& h) {
  T* d = nullptr;
  HIP_OK(hipMalloc(&d, h.size() * sizeof(T)));
  HIP_OK(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
  return d;
}

template <typename T>
std::vector<T> to_host(const T* d, size_t n) {
  std::vector<T> h(n);
  HIP_OK(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
  return h;
}

std::vector<float> widen(const std::vector<uint16_t>& h) {
  std::vector<float> f(h.size());
  orc_f16_to_f32_n(h.data(), f.data(), h.size());
  return f;
}

}  // namespace

int main(int argc, char** argv) {
  const int n_seqs = argc > 1 ? std::atoi(argv[1]) : 64;
  const uint64_t seed = argc > 2 ? std::strtoull(argv[2], nullptr, 10) : 1;
  const int q_heads = 14, kv_heads = 2, hd = 64, bs = 16, num_blocks = 32768;
  const int kv_dim = kv_heads * hd, q_dim = q_heads * hd;
  const int64_t slots_total = static_cast<int64_t>(num_blocks) * bs;
  std::mt19937_64 rng(seed);
  std::normal_distribution<float> normal(0.f, 1.f);
  std::uniform_real_distribution<double> uni(std::log(64.0), std::log(4096.0));

  // Contexts, fragmented tables, packed arrays (cuda_model.cu:434-491).
  std::vector<int> ctx(n_seqs), table_offset(n_seqs), tables, token_seq(n_seqs), token_pos(n_seqs);
  std::vector<int> perm(num_blocks);
  for (int i = 0; i < num_blocks; i++) perm[i] = i;
  std::shuffle(perm.begin(), perm.end(), rng);
  for (int s = 0; s < n_seqs; s++) {
    ctx[s] = static_cast<int>(std::lround(std::exp(uni(rng))));
    table_offset[s] = static_cast<int>(tables.size());
    const int nb = (ctx[s] + bs - 1) / bs;
    for (int b = 0; b < nb; b++) tables.push_back(perm[tables.size()]);
    token_seq[s] = s;
    token_pos[s] = ctx[s] - 1;
  }
  std::vector<int> slots(n_seqs);
  for (int s = 0; s < n_seqs; s++)
    slots[s] = static_cast<int>(orc_slot(tables.data() + table_offset[s], token_pos[s], bs));

  // fp16 values, rounded on the host by the oracle's rule (tensor.h:38-56).
  auto f16_normal = [&](size_t n) {
    std::vector<float> f(n);
    for (auto& x : f) x = normal(rng);
    std::vector<uint16_t> h(n);
    orc_f32_to_f16_n(f.data(), h.data(), n);
    return h;
  };
  std::vector<uint16_t> kc = f16_normal(static_cast<size_t>(slots_total) * kv_dim);
  std::vector<uint16_t> vc = f16_normal(static_cast<size_t>(slots_total) * kv_dim);
  std::vector<uint16_t> k_new = f16_normal(static_cast<size_t>(n_seqs) * kv_dim);
  std::vector<uint16_t> v_new = f16_normal(static_cast<size_t>(n_seqs) * kv_dim);
  std::vector<uint16_t> q = f16_normal(static_cast<size_t>(n_seqs) * q_dim);

  // Device side: the reference's call sequence of a decode step.
  __half* d_kc = reinterpret_cast<__half*>(to_device(kc));
  __half* d_vc = reinterpret_cast<__half*>(to_device(vc));
  __half* d_knew = reinterpret_cast<__half*>(to_device(k_new));
  __half* d_vnew = reinterpret_cast<__half*>(to_device(v_new));
  __half* d_q = reinterpret_cast<__half*>(to_device(q));
  int* d_slots = to_device(slots);
  int* d_tables = to_device(tables);
  int* d_toff = to_device(table_offset);
  int* d_tseq = to_device(token_seq);
  int* d_tpos = to_device(token_pos);
  __half *d_out1 = nullptr, *d_out2 = nullptr;
  HIP_OK(hipMalloc(&d_out1, static_cast<size_t>(n_seqs) * q_dim * 2));
  HIP_OK(hipMalloc(&d_out2, static_cast<size_t>(n_seqs) * q_dim * 2));
  const size_t ws_bytes = le_attention_decode_workspace_size(n_seqs, q_heads, kv_heads, hd);
  void* ws = nullptr;
  HIP_OK(hipMalloc(&ws, ws_bytes));
  HIP_OK(hipMemset(ws, 0, ws_bytes));
  engine::le_bridge_set_workspace(ws, ws_bytes);
  engine::le_bridge_set_cache_slots(slots_total);
  const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
  hipStream_t stream = nullptr;  // the reference launches on the default stream

  engine::launch_store_kv(d_knew, d_vnew, d_slots, d_kc, d_vc, n_seqs, kv_dim, stream);
  engine::launch_attention_decode(d_q, d_kc, d_vc, d_tables, d_toff, d_tseq, d_tpos, d_out1, n_seqs, q_heads,
                                  kv_heads, hd, bs, scale, stream);
  engine::launch_attention_decode_gqa(d_q, d_kc, d_vc, d_tables, d_toff, d_tseq, d_tpos, d_out2, n_seqs,
                                      q_heads, kv_heads, hd, bs, scale, stream);
  HIP_OK(hipDeviceSynchronize());
  bool threw = false;
  try {
    engine::launch_attention_decode_gqa(d_q, d_kc, d_vc, d_tables, d_toff, d_tseq, d_tpos, d_out2, n_seqs,
                                        q_heads, kv_heads, 96, bs, scale, stream);
  } catch (const std::runtime_error&) {
    threw = true;
  }

  // Host side: the oracle's scatter and attention on the same values.
  for (int s = 0; s < n_seqs; s++) {
    std::memcpy(&kc[static_cast<size_t>(slots[s]) * kv_dim], &k_new[static_cast<size_t>(s) * kv_dim], kv_dim * 2);
    std::memcpy(&vc[static_cast<size_t>(slots[s]) * kv_dim], &v_new[static_cast<size_t>(s) * kv_dim], kv_dim * 2);
  }
  const bool caches_equal = to_host(reinterpret_cast<uint16_t*>(d_kc), kc.size()) == kc &&
                            to_host(reinterpret_cast<uint16_t*>(d_vc), vc.size()) == vc;
  const std::vector<float> kf = widen(kc), vf = widen(vc), qf = widen(q);
  std::vector<float> want(static_cast<size_t>(n_seqs) * q_dim);
  orc_paged_attention(qf.data(), q_dim, kf.data(), vf.data(), tables.data(), table_offset.data(),
                      token_seq.data(), token_pos.data(), n_seqs, q_heads, kv_heads, hd, bs, scale, want.data(),
                      q_dim, 8);
  const std::vector<uint16_t> o1 = to_host(reinterpret_cast<uint16_t*>(d_out1), want.size());
  const std::vector<uint16_t> o2 = to_host(reinterpret_cast<uint16_t*>(d_out2), want.size());
  const std::vector<float> g1 = widen(o1);
  double err = 0.0;
  for (size_t i = 0; i < want.size(); i++) err = std::fmax(err, std::fabs(static_cast<double>(g1[i]) - want[i]));
  const double tol = 6e-4 + 4.0 * std::ldexp(1.0, -11);
  const bool same = o1 == o2;
  const bool ok = caches_equal && err < tol && same && threw;
  std::printf("bridge %s: n_seqs %d caches_equal %d max|err| %.3e (tol %.3e) decode==gqa %d throws %d\n",
              ok ? "ok" : "FAILED", n_seqs, caches_equal ? 1 : 0, err, tol, same ? 1 : 0, threw ? 1 : 0);
  for (void* p : {static_cast<void*>(d_kc), static_cast<void*>(d_vc), static_cast<void*>(d_knew),
                  static_cast<void*>(d_vnew), static_cast<void*>(d_q), static_cast<void*>(d_slots),
                  static_cast<void*>(d_tables), static_cast<void*>(d_toff), static_cast<void*>(d_tseq),
                  static_cast<void*>(d_tpos), static_cast<void*>(d_out1), static_cast<void*>(d_out2), ws})
    HIP_OK(hipFree(p));
  return ok ? 0 : 1;
}
