// bf16 MFMA GEMM for multi-token matmuls (prefill).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace th {

// Batches of at least this many tokens go to the MFMA GEMM.
constexpr size_t kGemmMinTokens = 16;

// Whether launch_gemm handles a [rows, cols] weight.
bool gemm_supported(size_t rows, size_t cols);

// out[t*rows + r] = w[r] . x[t] for t < n, on the matrix cores.
hipError_t launch_gemm(hipStream_t s, float *out, const uint16_t *w, size_t rows, size_t cols, const float *x,
                       size_t n);

}  // namespace th
