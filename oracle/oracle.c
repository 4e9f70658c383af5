/*
 * CPU oracle: TEST INFRASTRUCTURE ONLY (see oracle.h). Restates the reference
 * engine's fp32 CPU backend with identical loop and summation orders.
 *
 * Build flags matter for bit-identity: -ffp-contract=off (no fused
 * multiply-add, matching the reference built for baseline x86-64) and no
 * -ffast-math (no reassociation of the float sums).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------- tensor.h:20-28 ---------------- */
float orc_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t orc_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)(u >> 16); /* inf/nan kept, not rounded */
  const uint32_t lsb = (u >> 16) & 1u;
  return (uint16_t)((u + 0x7fffu + lsb) >> 16); /* round to nearest, ties to even */
}

void orc_f32_to_bf16_n(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_bf16(in[i]);
}

void orc_bf16_to_f32_n(const uint16_t* in, float* out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = orc_bf16_to_f32(in[i]);
}

/* ---------------- tensor.h:29-56 (fp16) ----------------
 * IEEE binary16 from binary32, round to nearest even: the result of
 * tensor.h's f32_to_f16 for every input (NaN becomes the quiet NaN with the
 * sign kept and payload 0x200). Written from the format: a normal result
 * rebiases the exponent and rounds the 13 dropped mantissa bits; a subnormal
 * result is the value in units of 2^-24, rounded. */
uint16_t orc_f32_to_f16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);  /* NaN */
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 (and inf): infinity */
  if (a <= 0x33000000u) return sign;                        /* <= 2^-25: zero (2^-25 ties to even 0) */
  if (a < 0x38800000u) {                                    /* below 2^-14: subnormal result */
    const uint32_t m = (a & 0x7fffffu) | 0x800000u;         /* 24-bit significand */
    const int shift = 126 - (int)(a >> 23);                 /* 14..24 */
    uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
    q += (rem > half || (rem == half && (q & 1u))) ? 1u : 0u;  /* may carry into the smallest normal */
    return (uint16_t)(sign | q);
  }
  const uint32_t r = a - 0x38000000u; /* exponent rebiased from 127 to 15 */
  uint32_t q = r >> 13;
  const uint32_t rem = r & 0x1fffu;
  q += (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ? 1u : 0u;
  return (uint16_t)(sign | q);
}

float orc_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  uint32_t u;
  if (e == 0) {
    const float v = (float)m * 0x1p-24f; /* exact: m < 2^10 */
    return sign ? -v : v;
  }
  if (e == 0x1f) u = sign | 0x7f800000u | (m << 13);
  else u = sign | ((e + 112u) << 23) | (m << 13);
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void orc_f32_to_f16_n(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = orc_f32_to_f16(in[i]);
}

void orc_f16_to_f32_n(const uint16_t* in, float* out, size_t n) {
  for (size_t i = 0; i < n; i++) out[i] = orc_f16_to_f32(in[i]);
}

/* ---------------- kv_cache.h:29-31 ---------------- */
int64_t orc_slot(const int32_t* blocks, int pos, int block_size) {
  return (int64_t)blocks[pos / block_size] * block_size + pos % block_size;
}

/* ---------------- cuda_model.cu:434-491 ----------------
 * flatten(): one entry per token in slice order; a logit row is the last token
 * of a slice with needs_logits. upload_step_indices(): sequences are numbered
 * in first-seen order, each distinct sequence's whole table is appended once,
 * table_offset[s] is where it starts, slots[t] = slot(pos) narrowed to int32. */
void orc_pack_step(const orc_slice* slices, int n_slices, int block_size, int32_t* token_ids,
                   int32_t* positions, int32_t* slots, int32_t* token_seq, int32_t* tables,
                   int32_t* table_offset, int32_t* logit_rows, int32_t counts_out[4]) {
  int32_t n = 0, ns = 0, nt = 0, nr = 0;
  int64_t* seen = (int64_t*)malloc(sizeof(int64_t) * (size_t)(n_slices > 0 ? n_slices : 1));
  int* seen_slice = (int*)malloc(sizeof(int) * (size_t)(n_slices > 0 ? n_slices : 1));
  for (int i = 0; i < n_slices; i++) {
    const orc_slice* sl = &slices[i];
    int idx = -1;
    for (int j = 0; j < ns; j++)
      if (seen[j] == sl->seq_key) { idx = j; break; }
    if (idx < 0) {
      idx = ns;
      seen[ns] = sl->seq_key;
      seen_slice[ns] = i;
      if (table_offset) table_offset[ns] = nt;
      if (tables)
        for (int b = 0; b < sl->num_blocks; b++) tables[nt + b] = sl->blocks[b];
      nt += sl->num_blocks;
      ns++;
    }
    for (int t = 0; t < sl->len; t++) {
      const int pos = sl->start + t;
      if (token_ids) token_ids[n] = sl->tokens[pos];
      if (positions) positions[n] = pos;
      if (token_seq) token_seq[n] = idx;
      if (slots) slots[n] = (int32_t)orc_slot(slices[seen_slice[idx]].blocks, pos, block_size);
      n++;
    }
    if (sl->needs_logits) {
      if (logit_rows) logit_rows[nr] = n - 1;
      nr++;
    }
  }
  free(seen);
  free(seen_slice);
  counts_out[0] = n;
  counts_out[1] = ns;
  counts_out[2] = nt;
  counts_out[3] = nr;
}

/* ---------------- store_kv.cu:20-36 / cpu_model.cpp:153-157 ---------------- */
void orc_store_kv(const float* k, const float* v, const int32_t* slots, float* k_cache,
                  float* v_cache, int n_tokens, int kv_dim) {
  for (int t = 0; t < n_tokens; t++) {
    memcpy(k_cache + (size_t)slots[t] * kv_dim, k + (size_t)t * kv_dim, sizeof(float) * kv_dim);
    memcpy(v_cache + (size_t)slots[t] * kv_dim, v + (size_t)t * kv_dim, sizeof(float) * kv_dim);
  }
}

void orc_store_kv_bf16(const float* k, const float* v, const int32_t* slots, uint16_t* k_cache,
                       uint16_t* v_cache, int n_tokens, int kv_dim) {
  for (int t = 0; t < n_tokens; t++) {
    orc_f32_to_bf16_n(k + (size_t)t * kv_dim, k_cache + (size_t)slots[t] * kv_dim, (size_t)kv_dim);
    orc_f32_to_bf16_n(v + (size_t)t * kv_dim, v_cache + (size_t)slots[t] * kv_dim, (size_t)kv_dim);
  }
}

/* ---------------- ops.h:87-111 ----------------
 * score_p = (sum_d q_d*k_d, d ascending, float) * scale; mx = running float max
 * from -inf; e_p = expf(score_p - mx); denom = sum e_p in double; out_d starts
 * at 0 and accumulates float(e_p/denom) * v_d in position order. */
#define ORC_ATTN_BODY(LOADK, LOADV)                                                        \
  const int kv_dim = kv_heads * head_dim;                                                  \
  float mx = -INFINITY;                                                                    \
  for (int p = 0; p <= pos; p++) {                                                         \
    const size_t base = (size_t)orc_slot(blocks, p, block_size) * kv_dim +                 \
                        (size_t)kv_head * head_dim;                                        \
    float s = 0.f;                                                                         \
    for (int d = 0; d < head_dim; d++) s += q[d] * LOADK(base + d);                        \
    s *= scale;                                                                            \
    scratch[p] = s;                                                                        \
    if (s > mx) mx = s;                                                                    \
  }                                                                                        \
  double denom = 0;                                                                        \
  for (int p = 0; p <= pos; p++) {                                                         \
    scratch[p] = expf(scratch[p] - mx);                                                    \
    denom += scratch[p];                                                                   \
  }                                                                                        \
  for (int d = 0; d < head_dim; d++) out[d] = 0.f;                                         \
  for (int p = 0; p <= pos; p++) {                                                         \
    const float w = (float)(scratch[p] / denom);                                           \
    const size_t base = (size_t)orc_slot(blocks, p, block_size) * kv_dim +                 \
                        (size_t)kv_head * head_dim;                                        \
    for (int d = 0; d < head_dim; d++) out[d] += w * LOADV(base + d);                      \
  }

void orc_paged_attention_head(const float* q, const float* k_cache, const float* v_cache,
                              const int32_t* blocks, int block_size, int pos, int kv_head,
                              int kv_heads, int head_dim, float scale, float* out,
                              float* scratch) {
#define LK(i) k_cache[i]
#define LV(i) v_cache[i]
  ORC_ATTN_BODY(LK, LV)
#undef LK
#undef LV
}

static void orc_paged_attention_head_bf16(const float* q, const uint16_t* k_cache,
                                          const uint16_t* v_cache, const int32_t* blocks,
                                          int block_size, int pos, int kv_head, int kv_heads,
                                          int head_dim, float scale, float* out, float* scratch) {
#define LK(i) orc_bf16_to_f32(k_cache[i])
#define LV(i) orc_bf16_to_f32(v_cache[i])
  ORC_ATTN_BODY(LK, LV)
#undef LK
#undef LV
}

static int max_pos_of(const int32_t* token_pos, int n) {
  int m = 0;
  for (int i = 0; i < n; i++)
    if (token_pos[i] > m) m = token_pos[i];
  return m;
}

/* cpu_model.cpp:160-185: one item per (token, head), kv_head = h / group. */
#define ORC_ATTN_LOOP(HEADFN)                                                                \
  const int group = q_heads / kv_heads;                                                      \
  const int64_t items = (int64_t)n_tokens * q_heads;                                         \
  const int mp = max_pos_of(token_pos, n_tokens);                                            \
  int nthr = threads > 1 ? threads : 1;                                                      \
  _Pragma("omp parallel num_threads(nthr)") {                                                \
    float* scratch = (float*)malloc(sizeof(float) * (size_t)(mp + 1));                       \
    _Pragma("omp for schedule(dynamic, 16)") for (int64_t w = 0; w < items; w++) {           \
      const int i = (int)(w / q_heads), h = (int)(w % q_heads);                              \
      HEADFN(q + (size_t)i * q_stride + (size_t)h * head_dim, k_cache, v_cache,              \
             tables + table_offset[token_seq[i]], block_size, token_pos[i], h / group,       \
             kv_heads, head_dim, scale, out + (size_t)i * out_stride + (size_t)h * head_dim, \
             scratch);                                                                       \
    }                                                                                        \
    free(scratch);                                                                           \
  }

void orc_paged_attention(const float* q, int q_stride, const float* k_cache, const float* v_cache,
                         const int32_t* tables, const int32_t* table_offset,
                         const int32_t* token_seq, const int32_t* token_pos, int n_tokens,
                         int q_heads, int kv_heads, int head_dim, int block_size, float scale,
                         float* out, int out_stride, int threads) {
  ORC_ATTN_LOOP(orc_paged_attention_head)
}

void orc_paged_attention_bf16kv(const float* q, int q_stride, const uint16_t* k_cache,
                                const uint16_t* v_cache, const int32_t* tables,
                                const int32_t* table_offset, const int32_t* token_seq,
                                const int32_t* token_pos, int n_tokens, int q_heads, int kv_heads,
                                int head_dim, int block_size, float scale, float* out,
                                int out_stride, int threads) {
  ORC_ATTN_LOOP(orc_paged_attention_head_bf16)
}

/* ---------------- ops.h:22-31 ---------------- */
void orc_rmsnorm(const float* x, const float* weight, float* out, int rows, int cols, float eps) {
  for (int r = 0; r < rows; r++) {
    const float* xr = x + (size_t)r * cols;
    float* o = out + (size_t)r * cols;
    double ss = 0;
    for (int i = 0; i < cols; i++) ss += (double)xr[i] * xr[i];
    const float inv = 1.0f / sqrtf((float)(ss / cols) + eps);
    for (int i = 0; i < cols; i++) o[i] = xr[i] * inv * weight[i];
  }
}

/* ---------------- ops.h:37-50 ---------------- */
void orc_rope_tables(int head_dim, int max_positions, float theta, float* cos_t, float* sin_t) {
  const int half = head_dim / 2;
  for (int i = 0; i < half; i++) {
    const double inv_freq = 1.0 / pow((double)theta, (2.0 * i) / head_dim);
    for (int p = 0; p < max_positions; p++) {
      const double angle = p * inv_freq;
      cos_t[(size_t)p * half + i] = (float)cos(angle);
      sin_t[(size_t)p * half + i] = (float)sin(angle);
    }
  }
}

/* ---------------- ops.h:55-66 (rotate_half pairing i <-> i+half) ---------------- */
void orc_rope_inplace(float* x, int heads, int head_dim, int pos, const float* cos_t,
                      const float* sin_t) {
  const int half = head_dim / 2;
  const float* c = cos_t + (size_t)pos * half;
  const float* s = sin_t + (size_t)pos * half;
  for (int h = 0; h < heads; h++) {
    float* v = x + (size_t)h * head_dim;
    for (int i = 0; i < half; i++) {
      const float a = v[i], b = v[i + half];
      v[i] = a * c[i] - b * s[i];
      v[i + half] = b * c[i] + a * s[i];
    }
  }
}

/* ---------------- ops.h:69-74 ---------------- */
void orc_silu_mul(float* gate, const float* up, size_t n) {
  for (size_t i = 0; i < n; i++) {
    const float g = gate[i];
    gate[i] = g / (1.0f + expf(-g)) * up[i];
  }
}

/* ---------------- sampler.cpp:9-13 (first maximum wins) ---------------- */
int32_t orc_argmax(const float* logits, int vocab) {
  int32_t best = 0;
  for (int i = 1; i < vocab; i++)
    if (logits[i] > logits[best]) best = i;
  return best;
}

/* ---------------- cpu_model.cpp:27-39 (naive branch) ----------------
 * C[i][j] = sum_t A[i][t]*B[j][t], t ascending, float accumulator starting at 0,
 * then C += bias[j]. The tiled kernel below keeps exactly that per-output order
 * (each output is its own accumulator lane; only different outputs are
 * computed side by side), so it is bit-identical to the naive triple loop. */
typedef float v8f __attribute__((vector_size(32)));

#define TI 4
#define TJ 16

__attribute__((target_clones("avx2", "default"))) static void linear_tile(
    const float* A, int k, const float* Bt, int n, int i0, int mi, int j0, float* C) {
  v8f acc[TI][2];
  for (int r = 0; r < TI; r++) acc[r][0] = acc[r][1] = (v8f){0, 0, 0, 0, 0, 0, 0, 0};
  for (int t = 0; t < k; t++) {
    v8f b0, b1;
    memcpy(&b0, Bt + (size_t)t * n + j0, 32);
    memcpy(&b1, Bt + (size_t)t * n + j0 + 8, 32);
    for (int r = 0; r < TI; r++) {
      const float a = A[(size_t)(i0 + (r < mi ? r : 0)) * k + t];
      const v8f av = {a, a, a, a, a, a, a, a};
      acc[r][0] = acc[r][0] + av * b0;
      acc[r][1] = acc[r][1] + av * b1;
    }
  }
  for (int r = 0; r < mi; r++) {
    memcpy(C + (size_t)(i0 + r) * n + j0, &acc[r][0], 32);
    memcpy(C + (size_t)(i0 + r) * n + j0 + 8, &acc[r][1], 32);
  }
}

void orc_linear(const float* A, int m, int k, const float* B, int n, const float* bias, float* C,
                int threads) {
  const int nthr = threads > 1 ? threads : 1;
  const int nj = n / TJ * TJ;
  if (nj > 0) {
    /* Transposed copy of B's first nj rows, so TJ consecutive outputs are one vector load. */
    float* Bt = (float*)malloc(sizeof(float) * (size_t)k * nj);
#pragma omp parallel for num_threads(nthr) schedule(static)
    for (int t = 0; t < k; t++)
      for (int j = 0; j < nj; j++) Bt[(size_t)t * nj + j] = B[(size_t)j * k + t];
    float* Ct = (float*)malloc(sizeof(float) * (size_t)m * nj);
    const int ntiles_i = (m + TI - 1) / TI, ntiles_j = nj / TJ;
#pragma omp parallel for num_threads(nthr) schedule(dynamic, 4) collapse(2)
    for (int tj = 0; tj < ntiles_j; tj++)
      for (int ti = 0; ti < ntiles_i; ti++) {
        const int i0 = ti * TI, mi = (m - i0) < TI ? (m - i0) : TI;
        linear_tile(A, k, Bt, nj, i0, mi, tj * TJ, Ct);
      }
    for (int i = 0; i < m; i++)
      memcpy(C + (size_t)i * n, Ct + (size_t)i * nj, sizeof(float) * nj);
    free(Ct);
    free(Bt);
  }
  /* Remaining columns: the reference's naive loop as written. */
#pragma omp parallel for num_threads(nthr) schedule(static)
  for (int i = 0; i < m; i++)
    for (int j = nj; j < n; j++) {
      const float* a = A + (size_t)i * k;
      const float* b = B + (size_t)j * k;
      float s = 0.f;
      for (int t = 0; t < k; t++) s += a[t] * b[t];
      C[(size_t)i * n + j] = s;
    }
  if (bias)
    for (int i = 0; i < m; i++)
      for (int j = 0; j < n; j++) C[(size_t)i * n + j] += bias[j];
}

/* ---------------- cpu_model.cpp:98-214 ---------------- */
void orc_forward_trace(const orc_model* m, const float* rope_cos, const float* rope_sin,
                       void* const* k_caches, void* const* v_caches, int kv_bf16,
                       const int32_t* token_ids, const int32_t* positions, const int32_t* slots,
                       const int32_t* token_seq, const int32_t* tables,
                       const int32_t* table_offset, int n_tokens, const int32_t* logit_rows,
                       int n_logits, int block_size, float* logits, int threads, float* resid) {
  const int N = n_tokens, H = m->hidden, hd = m->head_dim, nh = m->q_heads, nkv = m->kv_heads,
            I = m->inter, kv_dim = nkv * hd;
  const float scale = 1.0f / sqrtf((float)hd);
  memset(logits, 0, sizeof(float) * (size_t)n_logits * m->vocab);
  if (N == 0) return;

  float* x = (float*)malloc(sizeof(float) * (size_t)N * H);
  float* h = (float*)malloc(sizeof(float) * (size_t)N * H);
  float* q = (float*)malloc(sizeof(float) * (size_t)N * nh * hd);
  float* k = (float*)malloc(sizeof(float) * (size_t)N * kv_dim);
  float* v = (float*)malloc(sizeof(float) * (size_t)N * kv_dim);
  float* attn = (float*)malloc(sizeof(float) * (size_t)N * nh * hd);
  float* o = (float*)malloc(sizeof(float) * (size_t)N * H);
  float* gate = (float*)malloc(sizeof(float) * (size_t)N * I);
  float* up = (float*)malloc(sizeof(float) * (size_t)N * I);

  for (int i = 0; i < N; i++)
    memcpy(x + (size_t)i * H, m->embed + (size_t)token_ids[i] * H, sizeof(float) * H);
  /* The residual stream after the embedding and after every layer, as the
   * reference's per-layer capture records it (test_cpu_model.cpp:112-125). */
  if (resid) memcpy(resid, x, sizeof(float) * (size_t)N * H);

  const int QD = nh * hd;
  for (int l = 0; l < m->layers; l++) {
    orc_rmsnorm(x, m->in_norm[l], h, N, H, m->eps);
    orc_linear(h, N, H, m->wq[l], QD, m->bq ? m->bq[l] : NULL, q, threads);
    orc_linear(h, N, H, m->wk[l], kv_dim, m->bk ? m->bk[l] : NULL, k, threads);
    orc_linear(h, N, H, m->wv[l], kv_dim, m->bv ? m->bv[l] : NULL, v, threads);
    /* Rotate and write every token's K/V before any attention runs (cpu_model.cpp:144-158). */
    for (int i = 0; i < N; i++) {
      orc_rope_inplace(q + (size_t)i * QD, nh, hd, positions[i], rope_cos, rope_sin);
      orc_rope_inplace(k + (size_t)i * kv_dim, nkv, hd, positions[i], rope_cos, rope_sin);
    }
    if (kv_bf16) {
      orc_store_kv_bf16(k, v, slots, (uint16_t*)k_caches[l], (uint16_t*)v_caches[l], N, kv_dim);
      orc_paged_attention_bf16kv(q, QD, (const uint16_t*)k_caches[l],
                                 (const uint16_t*)v_caches[l], tables, table_offset, token_seq,
                                 positions, N, nh, nkv, hd, block_size, scale, attn, QD, threads);
    } else {
      orc_store_kv(k, v, slots, (float*)k_caches[l], (float*)v_caches[l], N, kv_dim);
      orc_paged_attention(q, QD, (const float*)k_caches[l], (const float*)v_caches[l], tables,
                          table_offset, token_seq, positions, N, nh, nkv, hd, block_size, scale,
                          attn, QD, threads);
    }
    orc_linear(attn, N, QD, m->wo[l], H, NULL, o, threads);
    for (size_t i = 0; i < (size_t)N * H; i++) x[i] += o[i];
    orc_rmsnorm(x, m->post_norm[l], h, N, H, m->eps);
    orc_linear(h, N, H, m->wgate[l], I, NULL, gate, threads);
    orc_linear(h, N, H, m->wup[l], I, NULL, up, threads);
    orc_silu_mul(gate, up, (size_t)N * I);
    orc_linear(gate, N, I, m->wdown[l], H, NULL, o, threads);
    for (size_t i = 0; i < (size_t)N * H; i++) x[i] += o[i];
    if (resid) memcpy(resid + (size_t)(l + 1) * N * H, x, sizeof(float) * (size_t)N * H);
  }

  if (n_logits > 0) {
    for (int r = 0; r < n_logits; r++)
      orc_rmsnorm(x + (size_t)logit_rows[r] * H, m->final_norm, h + (size_t)r * H, 1, H, m->eps);
    const float* head = m->tie_word_embeddings ? m->embed : m->lm_head;
    orc_linear(h, n_logits, H, head, m->vocab, NULL, logits, threads);
  }
  free(x); free(h); free(q); free(k); free(v); free(attn); free(o); free(gate); free(up);
}

void orc_forward(const orc_model* m, const float* rope_cos, const float* rope_sin,
                 void* const* k_caches, void* const* v_caches, int kv_bf16,
                 const int32_t* token_ids, const int32_t* positions, const int32_t* slots,
                 const int32_t* token_seq, const int32_t* tables, const int32_t* table_offset,
                 int n_tokens, const int32_t* logit_rows, int n_logits, int block_size,
                 float* logits, int threads) {
  orc_forward_trace(m, rope_cos, rope_sin, k_caches, v_caches, kv_bf16, token_ids, positions,
                    slots, token_seq, tables, table_offset, n_tokens, logit_rows, n_logits,
                    block_size, logits, threads, NULL);
}
