// Device model and serving loop over the hot path (le_engine.h).
//
// The forward pass follows the reference's CudaModel::forward
// (src/model/cuda/cuda_model.cu:324-429) and its CPU twin cpu_model.cpp:98-214:
// embedding gather, then per layer RMSNorm, Q/K/V projections (+bias),
// RoPE, the K/V scatter into the paged cache, ragged paged attention over the
// packed step, output projection and residual, RMSNorm, SiLU-gated MLP and
// residual; finally RMSNorm and the LM head on the logit rows only. Where the
// reference uploads six index arrays with synchronous copies every step, here
// the step is packed once (le_plan_step) and sent with one async copy, and
// greedy selection runs on the device so only the chosen ids come back.
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <new>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "../le_internal.h"
#include "le_engine.h"
#include "llm_engine_amd.h"
#include "model_kernels.h"
#include "scheduler.h"

namespace le::engine {
namespace {

// Graph-replayed steps use the fixed layout, where every row owns the same
// number of partition slots whatever its length, and empty slots still cost
// a workgroup. The partition is chosen per row count so that rows x slots x
// kv heads is about one workgroup per CU (a TinyLlama-shaped step, 64 rows of
// 128-1280 keys, 4 kv heads: one slot per row 17.3 us per launch, two 19.8;
// the Qwen2.5-0.5B shape, 2 kv heads: two slots 13.8 us, one 15.6).
// A slot never spans more than kGraphMaxPartition keys, so a long row is
// still split when the model's maximum context is long.
constexpr int kGraphWorkgroups = 256;
constexpr int kGraphMaxPartition = 4096;
int graph_partition(int rows, int kv_heads, int cap_blocks, int bs) {
  const int max_pb = std::max(1, kGraphMaxPartition / bs);
  const int slots = std::max({1, kGraphWorkgroups / std::max(1, rows * kv_heads), (cap_blocks + max_pb - 1) / max_pb});
  return ((cap_blocks + slots - 1) / slots) * bs;
}

}  // namespace

// A failure that carries the status the C ABI returns for it: a HIP error
// code, LE_EDEVICE for rocBLAS, or the LE_E* code of an inner call.
struct StatusError : std::runtime_error {
  int status;
  StatusError(int st, const std::string& msg) : std::runtime_error(msg), status(st) {}
};

namespace {

void hip_ok(hipError_t e, const char* what) {
  if (e != hipSuccess) throw StatusError(static_cast<int>(e), std::string(what) + ": " + hipGetErrorString(e));
}
void blas_ok(rocblas_status s, const char* what) {
  if (s != rocblas_status_success)
    throw StatusError(LE_EDEVICE, std::string(what) + ": rocBLAS status " + std::to_string(static_cast<int>(s)));
}
void le_ok(int st, const char* what) {
  if (st != LE_OK) throw StatusError(st, std::string(what) + ": " + le_status_string(st));
}

uint16_t to_bf16(float f) {  // round to nearest even, inf/nan unrounded (tensor.h:23-28)
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u) return static_cast<uint16_t>(u >> 16);
  return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// Bumped whenever a step buffer moves: captured decode graphs hold the old
// addresses and are captured again.
struct Generation {
  uint64_t value = 0;
};

// Thrown by a step buffer that would have to grow while the step's stream is
// being captured (allocating and clearing memory are not capturable): the
// capture is abandoned and the step runs eagerly.
struct GrowthDuringCapture {};

// Device buffer that grows on demand and is then reused across steps.
struct DevBuf {
  void* p = nullptr;
  size_t cap = 0;
  Generation* gen = nullptr;
  const bool* capturing = nullptr;
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  ~DevBuf() { if (p) (void)hipFree(p); }
  void* get(size_t bytes, bool zero = false, hipStream_t s = nullptr) {
    if (bytes > cap) {
      if (capturing && *capturing) throw GrowthDuringCapture{};
      if (p) hip_ok(hipFree(p), "hipFree");
      p = nullptr;
      hip_ok(hipMalloc(&p, bytes), "hipMalloc");
      cap = bytes;
      if (gen) gen->value++;
      if (zero) hip_ok(hipMemsetAsync(p, 0, bytes, s), "hipMemsetAsync");
    }
    return p;
  }
};

struct HostBuf {
  void* p = nullptr;
  size_t cap = 0;
  Generation* gen = nullptr;
  HostBuf() = default;
  HostBuf(const HostBuf&) = delete;
  HostBuf& operator=(const HostBuf&) = delete;
  ~HostBuf() { if (p) (void)hipHostFree(p); }
  void* get(size_t bytes) {
    if (bytes > cap) {
      if (p) hip_ok(hipHostFree(p), "hipHostFree");
      p = nullptr;
      hip_ok(hipHostMalloc(&p, bytes, hipHostMallocDefault), "hipHostMalloc");
      cap = bytes;
      if (gen) gen->value++;
    }
    return p;
  }
};

// Per-layer weights on the device. Q, K and V are stacked into one
// [q_dim + 2*kv_dim][hidden] matrix and gate/up into one [2*inter][hidden]
// matrix, so each is a single GEMM whose output rows feed the fused
// bias/RoPE/cache-write and SiLU kernels directly.
struct Layer {
  void *wqkv = nullptr, *wo = nullptr, *wgate_up = nullptr, *wdown = nullptr;
  float *in_norm = nullptr, *post_norm = nullptr, *bqkv = nullptr;
};

}  // namespace

class Model {
 public:
  Model(const le_model_desc& d, int num_blocks, int block_size);
  ~Model();
  void forward(const le_step_slice* slices, int n_slices, int32_t* tokens_out, float* logits_out);
  void set_decode_graph(bool on) { graph_on_ = on; }
  void set_plan_flags(int flags) { plan_flags_ = flags; graphs_clear(); }
  int64_t graph_replays() const { return graph_replays_; }
  int64_t eager_fallbacks() const { return eager_fallbacks_; }
  int num_blocks() const { return num_blocks_; }
  double plan_seconds() const { return plan_seconds_; }
  int block_size() const { return bs_; }

 private:
  void* upload(const float* host, size_t n, bool as_bf16) { return upload_parts({{host, n}}, as_bf16); }
  void* upload_parts(const std::vector<std::pair<const float*, size_t>>& parts, bool as_bf16);
  float* upload_f32(const float* host, size_t n) { return static_cast<float*>(upload(host, n, false)); }
  // C = A . B^T (accumulate: C += A . B^T, bf16 models only)
  void gemm(const void* A, const void* B, void* C, int m, int n, int k, bool c_f32 = false,
            bool accumulate = false);
  // The device work of a step on stream_, from the plan upload to the token
  // read-back into the pinned tokens buffer (nothing synchronises).
  void enqueue_step(le_step_plan& plan, const void* host_plan, float* logits_out);
  // Grows every step buffer enqueue_step uses to this plan's sizes (and
  // clears a new workspace), so that a capture of the same plan allocates
  // nothing.
  void size_buffers(const le_step_plan& plan);
  bool forward_graph(const le_step_slice* slices, int n_slices, int32_t* tokens_out);
  // The captured-graph path is not available: this step and every later one
  // run eagerly.
  void eager_fallback(le_step_plan& plan, const void* host, int n_slices, int32_t* tokens_out);
  void graphs_clear();

  le_model_desc d_;
  bool bf16_;
  // bf16 models: the post-attention RMSNorm folded around the gate|up
  // projection (its weight in the projection's columns, the residual add in
  // the O projection's epilogue, the row scale in rms_silu_mul): one launch
  // fewer per layer. fp32 models keep the reference's order of operations.
  bool fused_post_norm_ = false;
  // bf16 models with the ragged attention: the pre-attention RMSNorm folded
  // into the QKV projection as well (its weight in the projection's columns,
  // the row scale applied by le_ragged_paged_attention_qkv_rms, the residual
  // add in the down projection's epilogue): no norm launch inside a layer.
  bool fused_pre_norm_ = false;
  int kv_dt_;  // le_dtype of the caches
  double plan_seconds_ = 0.0;
  int H_, QD_, KVD_, I_, V_, hd_, nh_, nkv_, bs_, num_blocks_;
  size_t act_;
  hipStream_t stream_ = nullptr;
  rocblas_handle blas_ = nullptr;
  std::vector<void*> owned_;
  void* embed_ = nullptr;
  void* lm_head_ = nullptr;
  float* final_norm_ = nullptr;
  float *cos_ = nullptr, *sin_ = nullptr;
  std::vector<Layer> layers_;
  std::vector<void*> kc_, vc_;
  DevBuf x_, h_, qkv_, q_, attn_, o_, gate_up_, act_buf_, logits_, tokens_, plan_dev_, ws_;
  HostBuf plan_host_, tokens_host_;
  // The model launches on its own stream (no CU mask), where the XCD-local
  // exchange's precondition holds.
  int plan_flags_ = LE_PLAN_XCD_LOCAL;
  bool capturing_ = false;  // stream_ is being captured: step buffers must not grow
  // Decode graphs: per row count, the whole decode step captured once (after
  // one eager run of the same layout) and replayed while the buffers stay.
  struct DecodeGraph {
    hipGraphExec_t exec = nullptr;
    int64_t plan_bytes = 0;
    uint64_t gen = 0;
    bool warm = false;
  };
  Generation gen_;
  bool graph_on_ = false, graph_failed_ = false;
  int64_t graph_replays_ = 0, eager_fallbacks_ = 0;
  std::map<int, DecodeGraph> graphs_;
};

Model::Model(const le_model_desc& d, int num_blocks, int block_size) : d_(d) {
  bf16_ = d.dtype == LE_BF16;
  kv_dt_ = d.kv_dtype;
  if (d.dtype != LE_F32 && d.dtype != LE_BF16)
    throw StatusError(LE_EUNSUPPORTED, "model dtype: fp32 or bf16 weights and activations");
  if (kv_dt_ != LE_F32 && kv_dt_ != LE_BF16 && kv_dt_ != LE_F16) throw std::invalid_argument("kv_dtype");
  if (d.attention != LE_ATTN_RAGGED && d.attention != LE_ATTN_REFERENCE) throw std::invalid_argument("attention");
  H_ = d.hidden;
  hd_ = d.head_dim;
  nh_ = d.q_heads;
  nkv_ = d.kv_heads;
  QD_ = nh_ * hd_;
  KVD_ = nkv_ * hd_;
  I_ = d.inter;
  V_ = d.vocab;
  bs_ = block_size;
  num_blocks_ = num_blocks;
  act_ = bf16_ ? 2 : 4;
  fused_post_norm_ = bf16_ && !d.unfused_norms && rms_silu_mul_fits(H_, I_);
  fused_pre_norm_ = fused_post_norm_ && d.attention == LE_ATTN_RAGGED && H_ % 8 == 0;
  if (nh_ % nkv_ != 0 || hd_ % 2 != 0) throw std::invalid_argument("head layout");
  for (DevBuf* b : {&x_, &h_, &qkv_, &q_, &attn_, &o_, &gate_up_, &act_buf_, &logits_, &tokens_, &plan_dev_, &ws_}) {
    b->gen = &gen_;
    b->capturing = &capturing_;
  }
  for (HostBuf* b : {&plan_host_, &tokens_host_}) b->gen = &gen_;
  hip_ok(hipStreamCreate(&stream_), "hipStreamCreate");
  blas_ok(rocblas_create_handle(&blas_), "rocblas_create_handle");
  blas_ok(rocblas_set_stream(blas_, stream_), "rocblas_set_stream");

  embed_ = upload(d.embed, static_cast<size_t>(V_) * H_, bf16_);
  lm_head_ = d.tie_word_embeddings ? embed_ : upload(d.lm_head, static_cast<size_t>(V_) * H_, bf16_);
  final_norm_ = upload_f32(d.final_norm, H_);
  layers_.resize(d.layers);
  for (int l = 0; l < d.layers; l++) {
    Layer& L = layers_[l];
    L.in_norm = upload_f32(d.in_norm[l], H_);
    L.post_norm = upload_f32(d.post_norm[l], H_);
    const size_t hq = static_cast<size_t>(QD_) * H_, hkv = static_cast<size_t>(KVD_) * H_;
    if (fused_pre_norm_) {
      // q, k, v columns times the pre-attention norm weight, in fp32, then
      // rounded to bf16 once
      if (!d.wq[l] || !d.wk[l] || !d.wv[l] || !d.in_norm[l]) throw std::invalid_argument("missing weight");
      auto fold = [&](const float* w, size_t rows) {
        std::vector<float> f(rows * H_);
        for (size_t j = 0; j < rows; j++)
          for (size_t k = 0; k < static_cast<size_t>(H_); k++) f[j * H_ + k] = w[j * H_ + k] * d.in_norm[l][k];
        return f;
      };
      const std::vector<float> fq = fold(d.wq[l], QD_), fk = fold(d.wk[l], KVD_), fv = fold(d.wv[l], KVD_);
      L.wqkv = upload_parts({{fq.data(), hq}, {fk.data(), hkv}, {fv.data(), hkv}}, true);
    } else {
      L.wqkv = upload_parts({{d.wq[l], hq}, {d.wk[l], hkv}, {d.wv[l], hkv}}, bf16_);
    }
    L.wo = upload(d.wo[l], static_cast<size_t>(H_) * QD_, bf16_);
    if (d.bq && d.bq[l])
      L.bqkv = static_cast<float*>(upload_parts(
          {{d.bq[l], static_cast<size_t>(QD_)}, {d.bk[l], static_cast<size_t>(KVD_)},
           {d.bv[l], static_cast<size_t>(KVD_)}}, false));
    const size_t hi = static_cast<size_t>(I_) * H_;
    if (fused_post_norm_) {
      // gate|up columns times the post-attention norm weight, in fp32, then
      // rounded to bf16 once
      if (!d.wgate[l] || !d.wup[l] || !d.post_norm[l]) throw std::invalid_argument("missing weight");
      std::vector<float> g(hi), u(hi);
      for (size_t j = 0; j < static_cast<size_t>(I_); j++)
        for (size_t k = 0; k < static_cast<size_t>(H_); k++) {
          g[j * H_ + k] = d.wgate[l][j * H_ + k] * d.post_norm[l][k];
          u[j * H_ + k] = d.wup[l][j * H_ + k] * d.post_norm[l][k];
        }
      L.wgate_up = upload_parts({{g.data(), hi}, {u.data(), hi}}, true);
    } else {
      L.wgate_up = upload_parts({{d.wgate[l], hi}, {d.wup[l], hi}}, bf16_);
    }
    L.wdown = upload(d.wdown[l], static_cast<size_t>(H_) * I_, bf16_);
  }
  // RoPE tables as the reference builds them: angles in double, stored as
  // float (ops.h:37-50).
  const int half = hd_ / 2;
  std::vector<float> c(static_cast<size_t>(d.max_pos) * half), s(c.size());
  for (int i = 0; i < half; i++) {
    const double inv_freq = 1.0 / std::pow(static_cast<double>(d.theta), (2.0 * i) / hd_);
    for (int p = 0; p < d.max_pos; p++) {
      c[static_cast<size_t>(p) * half + i] = static_cast<float>(std::cos(p * inv_freq));
      s[static_cast<size_t>(p) * half + i] = static_cast<float>(std::sin(p * inv_freq));
    }
  }
  cos_ = upload_f32(c.data(), c.size());
  sin_ = upload_f32(s.data(), s.size());
  // Every layer's K and V pool in one allocation: the decode attention's
  // block gathers ran faster over pools carved from one large allocation
  // than over one allocation per pool (64 x 4096 rows over 268 MB pools:
  // 28.0 against 28.5 us per launch; the end-to-end decode leg's 42 MB pools
  // show no difference).
  const size_t cache_bytes = static_cast<size_t>(num_blocks) * bs_ * KVD_ * (kv_dt_ == LE_F32 ? 4 : 2);
  const size_t arena_bytes = 2 * cache_bytes * static_cast<size_t>(d.layers);
  void* arena = nullptr;
  hip_ok(hipMalloc(&arena, arena_bytes), "hipMalloc kv");
  owned_.push_back(arena);
  hip_ok(hipMemsetAsync(arena, 0, arena_bytes, stream_), "memset kv");
  for (int l = 0; l < d.layers; l++) {
    char* base = static_cast<char*>(arena) + 2 * cache_bytes * static_cast<size_t>(l);
    kc_.push_back(base);
    vc_.push_back(base + cache_bytes);
  }
  hip_ok(hipStreamSynchronize(stream_), "sync");
}

void Model::graphs_clear() {
  for (auto& [n, g] : graphs_)
    if (g.exec) (void)hipGraphExecDestroy(g.exec);
  graphs_.clear();
}

Model::~Model() {
  (void)hipStreamSynchronize(stream_);
  graphs_clear();
  for (void* p : owned_) (void)hipFree(p);
  if (blas_) rocblas_destroy_handle(blas_);
  if (stream_) (void)hipStreamDestroy(stream_);
}

// One device allocation holding the parts back to back (stacked matrices).
void* Model::upload_parts(const std::vector<std::pair<const float*, size_t>>& parts, bool as_bf16) {
  size_t n = 0;
  for (const auto& [host, cnt] : parts) {
    if (!host) throw std::invalid_argument("missing weight");
    n += cnt;
  }
  const size_t esz = as_bf16 ? 2 : 4;
  void* p = nullptr;
  hip_ok(hipMalloc(&p, n * esz), "hipMalloc weight");
  owned_.push_back(p);
  size_t off = 0;
  for (const auto& [host, cnt] : parts) {
    char* dst = static_cast<char*>(p) + off * esz;
    if (as_bf16) {
      std::vector<uint16_t> b(cnt);
      for (size_t i = 0; i < cnt; i++) b[i] = to_bf16(host[i]);
      hip_ok(hipMemcpy(dst, b.data(), cnt * 2, hipMemcpyHostToDevice), "upload");
    } else {
      hip_ok(hipMemcpy(dst, host, cnt * 4, hipMemcpyHostToDevice), "upload");
    }
    off += cnt;
  }
  return p;
}

// C[m][n] = A[m][k] * B[n][k]^T in row-major terms. rocBLAS is column-major,
// so it computes C^T = B * A^T: B with op T first, A with op N second.
void Model::gemm(const void* A, const void* B, void* C, int m, int n, int k, bool c_f32, bool accumulate) {
  const float one = 1.f, zero = 0.f;
  if (!bf16_) {
    if (accumulate) throw std::logic_error("accumulating GEMM on the fp32 model");
    blas_ok(rocblas_sgemm(blas_, rocblas_operation_transpose, rocblas_operation_none, n, m, k, &one,
                          static_cast<const float*>(B), k, static_cast<const float*>(A), k, &zero,
                          static_cast<float*>(C), n),
            "rocblas_sgemm");
    return;
  }
  const rocblas_datatype ct = c_f32 ? rocblas_datatype_f32_r : rocblas_datatype_bf16_r;
  blas_ok(rocblas_gemm_ex(blas_, rocblas_operation_transpose, rocblas_operation_none, n, m, k, &one,
                          B, rocblas_datatype_bf16_r, k, A, rocblas_datatype_bf16_r, k, accumulate ? &one : &zero,
                          C, ct, n,
                          C, ct, n, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0),
          "rocblas_gemm_ex");
}

void Model::forward(const le_step_slice* slices, int n_slices, int32_t* tokens_out, float* logits_out) {
  if (graph_on_ && !graph_failed_ && !logits_out && forward_graph(slices, n_slices, tokens_out)) return;
  const auto t_plan = std::chrono::steady_clock::now();
  le_plan_config cfg{nh_, nkv_, hd_, bs_, kv_dt_, 0, 0, 0, plan_flags_, 0};
  le_step_plan plan{};
  // Packed straight into the pinned buffer when it is large enough (one
  // call per step); sized first only when it must grow.
  void* host = plan_host_.p;
  int st = le_plan_step(slices, n_slices, &cfg, host, static_cast<int64_t>(plan_host_.cap), &plan);
  if (st == LE_ENOSPACE) {
    host = plan_host_.get(static_cast<size_t>(plan.bytes));
    st = le_plan_step(slices, n_slices, &cfg, host, plan.bytes, &plan);
  }
  le_ok(st, "le_plan_step");
  plan_seconds_ += std::chrono::duration<double>(std::chrono::steady_clock::now() - t_plan).count();
  if (plan.n_tokens == 0) return;
  enqueue_step(plan, host, logits_out);
  hip_ok(hipStreamSynchronize(stream_), "step sync");
  if (tokens_out && plan.n_logits > 0)
    std::memcpy(tokens_out, tokens_host_.p, static_cast<size_t>(plan.n_logits) * 4);
}

// A decode step (one row per sequence, every row sampled) replayed from a
// captured HIP graph: the plan is packed in the fixed layout for its row
// count (every table table_capacity entries, fixed partitions, fixed work
// lists), so the graph captured for that row count stays valid while the
// contexts grow; only the plan's contents change, in the same pinned buffer
// the graph's upload node reads. Returns false when the step is not a
// decode step (the caller runs it eagerly). Each row count runs once
// eagerly first, so every buffer has its size and rocBLAS its kernels
// before the capture.
bool Model::forward_graph(const le_step_slice* slices, int n_slices, int32_t* tokens_out) {
  if (n_slices <= 0) return false;
  for (int i = 0; i < n_slices; i++)
    if (slices[i].len != 1 || !slices[i].needs_logits) return false;
  const auto t_plan = std::chrono::steady_clock::now();
  const int cap_blocks = (d_.max_pos + bs_ - 1) / bs_;
  le_plan_config cfg{nh_, nkv_, hd_, bs_, kv_dt_, graph_partition(n_slices, nkv_, cap_blocks, bs_), 0, 0,
                     plan_flags_, cap_blocks};
  le_step_plan plan{};
  void* host = plan_host_.p;
  int st = le_plan_step(slices, n_slices, &cfg, host, static_cast<int64_t>(plan_host_.cap), &plan);
  if (st == LE_ENOSPACE) {
    host = plan_host_.get(static_cast<size_t>(plan.bytes));
    st = le_plan_step(slices, n_slices, &cfg, host, plan.bytes, &plan);
  }
  if (st != LE_OK) {  // e.g. a table longer than max_pos allows: run eagerly
    eager_fallbacks_++;
    return false;
  }
  DecodeGraph& g = graphs_[n_slices];
  plan_seconds_ += std::chrono::duration<double>(std::chrono::steady_clock::now() - t_plan).count();
  if (!g.warm || g.plan_bytes != plan.bytes) {  // first step of this layout: eager
    if (g.exec) (void)hipGraphExecDestroy(g.exec);
    g = DecodeGraph{};
    enqueue_step(plan, host, nullptr);
    hip_ok(hipStreamSynchronize(stream_), "step sync");
    g.warm = true;
    g.plan_bytes = plan.bytes;
  } else {
    if (!g.exec || g.gen != gen_.value) {
      if (g.exec) (void)hipGraphExecDestroy(g.exec);
      g.exec = nullptr;
      // Every buffer at its size before the capture, outside it.
      size_buffers(plan);
      hip_ok(hipStreamSynchronize(stream_), "sync");
      const uint64_t gen0 = gen_.value;
      hipGraph_t graph = nullptr;
      hip_ok(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
      capturing_ = true;
      bool grew = false;
      try {
        enqueue_step(plan, host, nullptr);
      } catch (const GrowthDuringCapture&) {
        grew = true;
      } catch (...) {
        capturing_ = false;
        (void)hipStreamEndCapture(stream_, &graph);
        if (graph) (void)hipGraphDestroy(graph);
        throw;
      }
      capturing_ = false;
      const hipError_t ec = hipStreamEndCapture(stream_, &graph);
      const hipError_t ei =
          ec == hipSuccess && !grew ? hipGraphInstantiate(&g.exec, graph, nullptr, nullptr, 0) : hipErrorUnknown;
      if (graph) (void)hipGraphDestroy(graph);
      if (ei != hipSuccess || gen_.value != gen0) {  // not capturable here: run every step eagerly
        if (g.exec) (void)hipGraphExecDestroy(g.exec);
        g.exec = nullptr;
        eager_fallback(plan, host, n_slices, tokens_out);
        return true;
      }
      g.gen = gen_.value;
    }
    hip_ok(hipGraphLaunch(g.exec, stream_), "hipGraphLaunch");
    hip_ok(hipStreamSynchronize(stream_), "step sync");
    graph_replays_++;
  }
  if (tokens_out) std::memcpy(tokens_out, tokens_host_.p, static_cast<size_t>(n_slices) * 4);
  return true;
}

void Model::eager_fallback(le_step_plan& plan, const void* host, int n_slices, int32_t* tokens_out) {
  graph_failed_ = true;
  eager_fallbacks_++;
  (void)hipGetLastError();
  enqueue_step(plan, host, nullptr);
  hip_ok(hipStreamSynchronize(stream_), "step sync");
  if (tokens_out) std::memcpy(tokens_out, tokens_host_.p, static_cast<size_t>(n_slices) * 4);
}

void Model::size_buffers(const le_step_plan& plan) {
  const size_t n = static_cast<size_t>(plan.n_tokens);
  const int QKV = QD_ + 2 * KVD_;
  plan_dev_.get(static_cast<size_t>(plan.bytes));
  x_.get(n * H_ * act_);
  h_.get(n * H_ * act_);
  qkv_.get(n * QKV * act_);
  q_.get(n * QD_ * act_);
  attn_.get(n * QD_ * act_);
  o_.get(n * H_ * act_);
  gate_up_.get(n * 2 * I_ * act_);
  act_buf_.get(n * I_ * act_);
  const size_t ws_bytes = d_.attention == LE_ATTN_REFERENCE
                              ? le_attention_decode_workspace_size(plan.n_tokens, nh_, nkv_, hd_)
                              : le_ragged_workspace_size(&plan);
  if (ws_bytes) ws_.get(ws_bytes, /*zero=*/true, stream_);
  const size_t R = static_cast<size_t>(plan.n_logits);
  if (R > 0) {
    logits_.get(R * V_ * 4);
    tokens_.get(R * 4);
    tokens_host_.get(R * 4);
  }
}

void Model::enqueue_step(le_step_plan& plan, const void* host_plan, float* logits_out) {
  le_ok(le_plan_upload(&plan, host_plan, plan_dev_.get(static_cast<size_t>(plan.bytes)), stream_), "le_plan_upload");
  const int N = plan.n_tokens, R = plan.n_logits;
  const int32_t* d_ids = le_plan_dev_array(&plan, plan.off_token_ids);
  const int32_t* d_rows = le_plan_dev_array(&plan, plan.off_logit_rows);
  const size_t n = static_cast<size_t>(N);
  const int QKV = QD_ + 2 * KVD_;
  void* x = x_.get(n * H_ * act_);
  void* h = h_.get(n * H_ * act_);
  void* qkv = qkv_.get(n * QKV * act_);
  void* q = q_.get(n * QD_ * act_);
  void* attn = attn_.get(n * QD_ * act_);
  void* o = o_.get(n * H_ * act_);
  void* gate_up = gate_up_.get(n * 2 * I_ * act_);
  void* act = act_buf_.get(n * I_ * act_);
  const bool ref_attn = d_.attention == LE_ATTN_REFERENCE;
  const size_t ws_bytes =
      ref_attn ? le_attention_decode_workspace_size(N, nh_, nkv_, hd_) : le_ragged_workspace_size(&plan);
  void* ws = ws_bytes ? ws_.get(ws_bytes, /*zero=*/true, stream_) : nullptr;
  const float scale = 1.0f / std::sqrt(static_cast<float>(hd_));
  const le_dtype act_dt = bf16_ ? LE_BF16 : LE_F32, kv_dt = static_cast<le_dtype>(kv_dt_);
  const int L_n = static_cast<int>(layers_.size());

  // Per layer: norm (fused with the previous residual add), one QKV GEMM,
  // attention with bias+RoPE+cache-write (inside its launch on a decode
  // step), O GEMM, residual+norm, one gate|up GEMM, SiLU product, down GEMM.
  hip_ok(gather_rows(embed_, d_ids, x, N, H_, bf16_, stream_), "embedding");
  if (!fused_pre_norm_)
    hip_ok(residual_rmsnorm(x, nullptr, nullptr, layers_[0].in_norm, h, N, H_, d_.eps, false, bf16_, stream_),
           "rmsnorm");
  for (int l = 0; l < L_n; l++) {
    const Layer& L = layers_[l];
    gemm(fused_pre_norm_ ? x : h, L.wqkv, qkv, N, QKV, H_);
    // Bias, RoPE, the K/V store and attention from the QKV rows: one launch
    // on a decode step; otherwise every token's K/V is rotated and written
    // before attention runs, so tokens of one step (a prefill chunk) attend
    // to each other.
    if (fused_pre_norm_) {
      le_ok(le_ragged_paged_attention_qkv_rms(qkv, act_dt, QKV, L.bqkv, x, H_, d_.eps, cos_, sin_, d_.max_pos,
                                              kc_[l], vc_[l], kv_dt, num_blocks_, &plan, scale, attn, q, ws,
                                              ws_bytes, stream_),
            "le_ragged_paged_attention_qkv_rms");
    } else if (!ref_attn) {
      le_ok(le_ragged_paged_attention_qkv(qkv, act_dt, QKV, L.bqkv, cos_, sin_, d_.max_pos, kc_[l], vc_[l],
                                          kv_dt, num_blocks_, &plan, scale, attn, q, ws, ws_bytes, stream_),
            "le_ragged_paged_attention_qkv");
    } else {
      // the reference's sequence: bias, RoPE and the K/V store, then its
      // attention launcher over the packed arrays (cuda_model.cu:358-377)
      const int32_t* pos = le_plan_dev_array(&plan, plan.off_positions);
      le_ok(le_rope_kv_cache_write(qkv, act_dt, QKV, L.bqkv, pos, le_plan_dev_array(&plan, plan.off_slots), cos_,
                                   sin_, d_.max_pos, N, nh_, nkv_, hd_, q, kc_[l], vc_[l], kv_dt,
                                   static_cast<int64_t>(num_blocks_) * bs_, stream_),
            "le_rope_kv_cache_write");
      le_ok(le_attention_decode(q, act_dt, kc_[l], vc_[l], kv_dt, le_plan_dev_array(&plan, plan.off_tables),
                                le_plan_dev_array(&plan, plan.off_table_offset),
                                le_plan_dev_array(&plan, plan.off_token_seq), pos, attn, N, nh_, nkv_, hd_, bs_, scale,
                                num_blocks_, ws, ws_bytes, stream_),
            "le_attention_decode");
    }
    if (fused_post_norm_) {
      gemm(attn, L.wo, x, N, H_, QD_, false, /*accumulate=*/true);  // x += o
      gemm(x, L.wgate_up, gate_up, N, 2 * I_, H_);
      hip_ok(rms_silu_mul(x, gate_up, act, N, H_, I_, d_.eps, stream_), "rms_silu_mul");
    } else {
      gemm(attn, L.wo, o, N, H_, QD_);
      hip_ok(residual_rmsnorm(x, o, nullptr, L.post_norm, h, N, H_, d_.eps, true, bf16_, stream_), "residual");
      gemm(h, L.wgate_up, gate_up, N, 2 * I_, H_);
      hip_ok(silu_mul_split(gate_up, act, N, I_, bf16_, stream_), "silu_mul");
    }
    if (fused_pre_norm_) {
      gemm(act, L.wdown, x, N, H_, I_, false, /*accumulate=*/true);  // x += down; the next norm is folded
    } else {
      gemm(act, L.wdown, o, N, H_, I_);
      if (l + 1 < L_n)
        hip_ok(residual_rmsnorm(x, o, nullptr, layers_[l + 1].in_norm, h, N, H_, d_.eps, true, bf16_, stream_),
               "residual");
    }
  }
  if (R > 0) {
    // The last residual add (already in x when the norms are folded) and the
    // final norm, on the logit rows only.
    hip_ok(residual_rmsnorm(x, fused_pre_norm_ ? nullptr : o, d_rows, final_norm_, h, R, H_, d_.eps, false, bf16_,
                            stream_),
           "final norm");
    float* logits = static_cast<float*>(logits_.get(static_cast<size_t>(R) * V_ * 4));
    gemm(h, lm_head_, logits, R, V_, H_, /*c_f32=*/true);
    int32_t* dtok = static_cast<int32_t*>(tokens_.get(static_cast<size_t>(R) * 4));
    hip_ok(argmax_rows(logits, R, V_, dtok, stream_), "argmax");
    int32_t* htok = static_cast<int32_t*>(tokens_host_.get(static_cast<size_t>(R) * 4));
    hip_ok(hipMemcpyAsync(htok, dtok, static_cast<size_t>(R) * 4, hipMemcpyDeviceToHost, stream_), "tokens");
    if (logits_out)
      hip_ok(hipMemcpyAsync(logits_out, logits, static_cast<size_t>(R) * V_ * 4, hipMemcpyDeviceToHost,
                            stream_), "logits");
  }
}


}  // namespace le::engine

using le::engine::Model;

struct le_model {
  std::unique_ptr<Model> impl;
};

namespace {
// The status of a failed call: the one the failure carries; a rejected
// argument (std::invalid_argument) or anything else is LE_EINVAL, host
// memory exhaustion LE_ENOSPACE.
int fail(const std::exception& e) {
  std::fprintf(stderr, "llm-engine-amd: %s\n", e.what());
  if (const auto* se = dynamic_cast<const le::engine::StatusError*>(&e)) return se->status;
  if (dynamic_cast<const std::bad_alloc*>(&e)) return LE_ENOSPACE;
  return LE_EINVAL;
}
}  // namespace

extern "C" {

le_model* le_model_create(const le_model_desc* desc, int num_blocks, int block_size, int* status) {
  if (status) *status = LE_OK;
  if (!desc || num_blocks <= 0 || block_size <= 0) {
    if (status) *status = LE_EINVAL;
    return nullptr;
  }
  try {
    auto* m = new le_model;
    m->impl = std::make_unique<Model>(*desc, num_blocks, block_size);
    return m;
  } catch (const std::exception& e) {
    if (status) *status = fail(e);
    return nullptr;
  }
}

void le_model_destroy(le_model* m) { delete m; }

int le_model_set_decode_graph(le_model* m, int enable) {
  if (!m) return LE_EINVAL;
  m->impl->set_decode_graph(enable != 0);
  return LE_OK;
}

int64_t le_model_graph_replays(const le_model* m) { return m ? m->impl->graph_replays() : 0; }

int le_model_set_plan_flags(le_model* m, int32_t flags) {
  if (!m) return LE_EINVAL;
  if ((flags & ~(LE_PLAN_TWO_LAUNCHES | LE_PLAN_XCD_LOCAL)) != 0) return LE_EINVAL;
  m->impl->set_plan_flags(flags);
  return LE_OK;
}

int64_t le_model_eager_fallbacks(const le_model* m) { return m ? m->impl->eager_fallbacks() : 0; }


int le_argmax_rows(const float* logits, int rows, int vocab, int32_t* out, hipStream_t stream) {
  if (rows < 0 || vocab <= 0) return LE_EINVAL;
  if (rows == 0) return LE_OK;
  if (!logits || !out) return LE_EINVAL;
  const hipError_t e = le::engine::argmax_rows(logits, rows, vocab, out, stream);
  return e == hipSuccess ? LE_OK : static_cast<int>(e);
}

int le_model_forward(le_model* m, const le_step_slice* slices, int n_slices, int32_t* tokens_out,
                     float* logits_out) {
  if (!m || (n_slices > 0 && !slices)) return LE_EINVAL;
  try {
    m->impl->forward(slices, n_slices, tokens_out, logits_out);
    return LE_OK;
  } catch (const std::exception& e) {
    return fail(e);
  }
}

int le_run_greedy(le_model* m, const le_sched_config* cfg, int prefix_caching, int fragment_blocks,
                  int n_seqs, const int32_t* prompt_lens, const int32_t* prompts_flat,
                  const int32_t* max_tokens, const double* arrival_s, int32_t* gen_out,
                  le_run_stats* stats) {
  using namespace le::engine;
  if (!m || !cfg || n_seqs < 0 || (n_seqs > 0 && (!prompt_lens || !prompts_flat || !max_tokens || !gen_out)))
    return LE_EINVAL;
  try {
    Model& model = *m->impl;
    KVCacheManager kv(model.num_blocks(), model.block_size(), prefix_caching != 0);
    // Pre-fragment or shuffle the pool (test_cuda_invariance.cpp:98-105).
    std::vector<BlockTable> held = prepare_pool(kv, fragment_blocks);

    SchedulerConfig sc;
    sc.continuous = cfg->continuous != 0;
    sc.max_num_seqs = cfg->max_num_seqs;
    sc.max_num_batched_tokens = cfg->max_num_batched_tokens;
    sc.prefill_chunk_size = cfg->prefill_chunk_size;
    sc.admission_lookahead = cfg->admission_lookahead;
    sc.starvation_wait_steps = cfg->starvation_wait_steps;
    sc.watermark_blocks = cfg->watermark_blocks;
    sc.max_queue_wait_seconds = cfg->max_queue_wait_seconds;
    Scheduler sch(sc, kv);

    std::vector<SequencePtr> seqs(static_cast<size_t>(n_seqs));
    size_t off = 0;
    for (int i = 0; i < n_seqs; i++) {
      auto s = std::make_shared<Sequence>();
      s->id = static_cast<uint64_t>(i);
      s->tokens.assign(prompts_flat + off, prompts_flat + off + prompt_lens[i]);
      off += static_cast<size_t>(prompt_lens[i]);
      s->prompt_len = prompt_lens[i];
      s->params.max_tokens = max_tokens[i];
      s->params.ignore_eos = true;
      seqs[i] = s;
    }
    std::vector<int> order(static_cast<size_t>(n_seqs));
    for (int i = 0; i < n_seqs; i++) order[i] = i;
    if (arrival_s)
      std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return arrival_s[a] < arrival_s[b]; });
    size_t next = 0;

    le_run_stats rs{};
    const double plan_s0 = model.plan_seconds();
    std::vector<double> first_tok(static_cast<size_t>(n_seqs), -1.0), last_tok(static_cast<size_t>(n_seqs), -1.0);
    const auto t0 = std::chrono::steady_clock::now();
    auto elapsed = [&]() { return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count(); };
    std::vector<le_step_slice> sl;
    std::vector<int32_t> sampled;
    for (int guard = 0; guard < 10000000; guard++) {
      const double now = elapsed();
      while (next < order.size() && (!arrival_s || arrival_s[order[next]] <= now)) sch.add(seqs[order[next++]]);
      if (!sch.has_work()) {
        if (next >= order.size()) break;
        const double wait = arrival_s[order[next]] - elapsed();
        if (wait > 0) std::this_thread::sleep_for(std::chrono::duration<double>(wait));
        continue;
      }
      StepInput step = sch.schedule();
      if (step.empty()) {
        if (next >= order.size() && !sch.has_work()) break;
        continue;
      }
      sl.clear();
      for (const auto& s : step.slices)
        sl.push_back({static_cast<int64_t>(s.seq->id), s.start, s.len, s.needs_logits ? 1 : 0,
                      s.seq->block_table.num_blocks(), s.seq->block_table.blocks.data(),
                      s.seq->tokens.data()});
      sampled.assign(static_cast<size_t>(step.num_logits), 0);
      const double ts = elapsed();
      model.forward(sl.data(), static_cast<int>(sl.size()), sampled.data(), nullptr);
      const double te = elapsed();
      if (step.num_prefill_tokens == 0) {
        rs.decode_seconds += te - ts;
        rs.decode_steps++;
        rs.decode_step_tokens += step.num_logits;
        for (const auto& s : step.slices) rs.decode_context_tokens += s.start + s.len;
      }
      rs.steps++;
      rs.prompt_tokens += step.num_prefill_tokens;
      rs.decode_tokens += step.num_logits;
      sch.on_step_done(step, sampled);
      for (const auto& s : step.slices) {
        if (!s.needs_logits) continue;
        const size_t i = static_cast<size_t>(s.seq->id);
        if (first_tok[i] < 0) first_tok[i] = te;
        last_tok[i] = te;
      }
    }
    rs.seconds = elapsed();
    int n_done = 0;
    for (int i = 0; i < n_seqs; i++) {
      if (first_tok[i] < 0) continue;
      const double arr = arrival_s ? arrival_s[i] : 0.0;
      rs.ttft_mean_s += first_tok[i] - arr;
      rs.latency_mean_s += last_tok[i] - arr;
      n_done++;
    }
    if (n_done) {
      rs.ttft_mean_s /= n_done;
      rs.latency_mean_s /= n_done;
    }
    rs.preemptions = static_cast<int64_t>(sch.stats().preemptions);
    rs.plan_seconds = model.plan_seconds() - plan_s0;
    for (BlockTable& bt : held) kv.free(bt);
    size_t out_off = 0;  // gen_out: max_tokens[i] entries per sequence, back to back
    for (int i = 0; i < n_seqs; i++) {
      const Sequence& s = *seqs[i];
      for (int j = 0; j < max_tokens[i]; j++)
        gen_out[out_off + j] = j < s.num_generated() ? s.tokens[s.prompt_len + j] : -1;
      out_off += static_cast<size_t>(max_tokens[i]);
    }
    if (stats) *stats = rs;
    return LE_OK;
  } catch (const std::exception& e) {
    return fail(e);
  }
}

}  // extern "C"
