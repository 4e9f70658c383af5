// Launchers of the device model's layer kernels (model_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace le::engine {

hipError_t gather_rows(const void* table, const int32_t* ids, void* out, int n, int cols, bool bf16,
                       hipStream_t s);
// x[r] += y[r] (y may be NULL), out[b] = rmsnorm(x[r]) * w with r = rows ? rows[b] : b.
hipError_t residual_rmsnorm(void* x, const void* y, const int32_t* rows, const float* w, void* out,
                            int n_out, int cols, float eps, bool write_x, bool bf16, hipStream_t s);
// act[t] = silu(gate_up[t][:inter]) * gate_up[t][inter:]
hipError_t silu_mul_split(const void* gate_up, void* act, int rows, int inter, bool bf16, hipStream_t s);
// bf16 rows: act[t] = silu(g r) * (u r), r = 1/sqrt(mean(x[t]^2) + eps), with
// g, u the halves of gate_up[t] (the post-attention norm folded around the
// gate|up projection, whose weight columns carry the norm weight).
bool rms_silu_mul_fits(int hidden, int inter);
hipError_t rms_silu_mul(const void* x, const void* gate_up, void* act, int rows, int hidden, int inter, float eps,
                        hipStream_t s);
hipError_t argmax_rows(const float* logits, int rows, int vocab, int32_t* out, hipStream_t s);

}  // namespace le::engine
