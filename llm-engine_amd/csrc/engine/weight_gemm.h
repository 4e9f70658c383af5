// Weight-streaming GEMM for decode steps (weight_gemm.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

namespace le::engine {

constexpr int kMaxGemmRows = 64;

// Y[m][n] = X[m][k] . W[n][k]^T, bf16 X and W (row-major), fp32 accumulation,
// for 1 <= m <= 64, k % 128 == 0, n % 64 == 0. silu: W = [gate; up] (n rows,
// n / 2 % 32 == 0) and Y[m][n/2] = silu(gate) * up (bf16). out_f32 selects an
// fp32 Y (not with silu). splits = 0 picks the k split; the workspace (zeroed
// once; every launch leaves it zeroed) holds split partials and counters.
bool weight_gemm_supported(int m, int k, int n, bool silu);
size_t weight_gemm_workspace(int m, int k, int n, bool silu, int splits);
hipError_t weight_gemm(const void* x, int m, int k, const void* w, int n, bool silu, void* out, bool out_f32,
                       void* ws, size_t ws_bytes, int splits, hipStream_t s);

}  // namespace le::engine
