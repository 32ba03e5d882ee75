// bf16 MFMA GEMM for multi-token matmuls (prefill).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include <algorithm>

namespace th {

// Batches of at least this many tokens go to the MFMA GEMM.
constexpr size_t kGemmMinTokens = 16;

// Whether launch_gemm handles a [rows, cols] weight.
bool gemm_supported(size_t rows, size_t cols);

// out[t*rows + r] = w[r] . x[t] for t < n, on the matrix cores.
hipError_t launch_gemm(hipStream_t s, float *out, const uint16_t *w, size_t rows, size_t cols, const float *x,
                       size_t n);

// One weight matrix of a multi-matrix GEMM: out[t*rows + r] = w[r] . x[t].
struct GemmOut {
    const uint16_t *w;
    size_t rows;
    float *out;
};

// launch_gemm for 1-3 matrices that share x (one GEMM launch over all their
// rows), with its scratch in stream-ordered memory for the call.
hipError_t launch_gemm_outs(hipStream_t s, const float *x, size_t n, size_t cols, const GemmOut *outs, int n_outs);

// Most ways a single-matrix GEMM splits its K range (into partial tiles that a
// second kernel sums in a fixed order).
constexpr int kGemmMaxSplitK = 4;

// split_bf16 of x [n][cols] into hi[n * cols], lo[n * cols].
hipError_t launch_gemm_split(hipStream_t s, const float *x, size_t n, size_t cols, uint16_t *hi, uint16_t *lo);

// Ways the GEMM of n tokens, `rows` output rows (all matrices) and `cols`
// columns splits K for n_outs matrices (1: no split).
int gemm_ksplit(size_t n, size_t rows, size_t cols, int n_outs);

// The GEMM on split activations hi/lo [n][cols]: with ksplit > 1 (one
// matrix) the partial products go to part[ksplit][n][rows] instead of the
// output, to be summed by the consumer in split order.
hipError_t launch_gemm_hl(hipStream_t s, const uint16_t *hi, const uint16_t *lo, size_t n, size_t cols,
                          const GemmOut *outs, int n_outs, float *part, int ksplit);

// The gate and up GEMMs on split activations hi/lo [n][cols] with the SiLU
// epilogue of model/cpu.rs:151-155: h = silu(x . gate) * (x . up) for the
// [inter, cols] gate and up, written as split_bf16 terms h_hi / h_lo
// [n][inter] (the down projection's GEMM input). inter % 64 == 0.
hipError_t launch_gemm_silu(hipStream_t s, const uint16_t *hi, const uint16_t *lo, size_t n, size_t cols,
                            const uint16_t *gate, const uint16_t *up, size_t inter, uint16_t *h_hi, uint16_t *h_lo);

// Whether the q/k/v GEMM of n tokens takes launch_gemm_qkv: head_dim 128 and
// a launch the large tile would not take.
bool gemm_qkv_fused(size_t n, size_t q_rows, size_t kv_rows, size_t cols, size_t head_dim);

// The q, k and v GEMMs on split activations hi/lo [a.n][cols] (weights
// [n_heads * 128, cols] and [n_kv_heads * 128, cols] x 2) with the
// post-processing of launch_qk_norm_rope_append in the epilogue: q heads
// RMSNorm'd and rotated into a.q, k heads RMSNorm'd, rotated and v heads
// copied into the caches at positions pos + t. a.k and a.v are unused.
struct QkvPostArgs;
hipError_t launch_gemm_qkv(hipStream_t s, const uint16_t *hi, const uint16_t *lo, size_t cols, const uint16_t *wq,
                           const uint16_t *wk, const uint16_t *wv, const QkvPostArgs &a);

// Whether the q/k/v GEMM of n tokens at host position pos takes
// launch_gemm_qkv_huge: head_dim 128, matrices of whole 256-row tiles, a
// launch the 256 x 256 tile takes, pos a multiple of 32.
bool gemm_qkv_huge_fused(size_t n, size_t q_rows, size_t kv_rows, size_t cols, size_t head_dim, long long pos);

// launch_gemm_qkv on the 256 x 256 tile (a.pos_dev null): the same
// post-processing, and with a.kh the planes of the new keys and values.
hipError_t launch_gemm_qkv_huge(hipStream_t s, const uint16_t *hi, const uint16_t *lo, size_t cols,
                                const uint16_t *wq, const uint16_t *wk, const uint16_t *wv, const QkvPostArgs &a);

// Bytes of scratch launch_gemm_multi needs for n tokens of `cols` columns and
// single-matrix outputs of up to `rows` rows (room for the split-K partials).
size_t gemm_scratch_bytes(size_t n, size_t cols, size_t rows);

// Up to three matrices that share the input x [n][cols], in two launches (the
// activation split into `scratch`, then one GEMM over all their rows); a
// single matrix of few row tiles may split K, with partials in the rest of
// `scratch` (scratch_bytes long) and a third launch that sums them.
hipError_t launch_gemm_multi(hipStream_t s, const float *x, size_t n, size_t cols, const GemmOut *outs, int n_outs,
                             void *scratch, size_t scratch_bytes);

}  // namespace th
