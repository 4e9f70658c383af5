// Launchers of the device model's layer kernels (model_kernels.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace le::engine {

hipError_t gather_rows(const void* table, const int32_t* ids, void* out, int n, int cols, bool bf16,
                       hipStream_t s);
hipError_t rmsnorm(const void* x, const float* w, void* out, int rows, int cols, float eps, bool bf16,
                   hipStream_t s);
hipError_t rope(void* x, const int32_t* positions, const float* cos_t, const float* sin_t, int n,
                int heads, int head_dim, int row_stride, bool bf16, hipStream_t s);
hipError_t silu_mul(void* gate, const void* up, int64_t n, bool bf16, hipStream_t s);
hipError_t add_inplace(void* x, const void* y, int64_t n, bool bf16, hipStream_t s);
hipError_t add_bias(void* x, const float* bias, int rows, int cols, bool bf16, hipStream_t s);
hipError_t argmax_rows(const float* logits, int rows, int vocab, int32_t* out, hipStream_t s);

}  // namespace le::engine
