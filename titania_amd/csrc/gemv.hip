// Device::matmul (model/cpu.rs:49-77): out[t][r] = w[r] . x[t] with bf16
// weights and f32 activations, fp32 accumulation.
//
// For the few-token case (decode, n <= 8 per pass) this is a bandwidth-bound
// GEMV: each wave owns ROWS weight rows, every lane streams 16-byte chunks
// (8 bf16) of each row, and a wave64 shuffle reduction finishes each dot
// product. Larger batches go to the MFMA GEMM (gemm.hip).
#include "common.h"
#include "device_util.h"
#include "gemm.h"

namespace th {

template <int ROWS, int NT>
__global__ __launch_bounds__(256) void gemv_kernel(float *__restrict__ out, const uint16_t *__restrict__ w,
                                                   size_t rows, size_t cols, const float *__restrict__ x,
                                                   int n, size_t out_stride) {
    const int lane = threadIdx.x & 63;
    const size_t r0 = ((size_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * ROWS;
    if (r0 >= rows) return;
    const size_t chunks = cols / 8;
    const uint4 *wr[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        size_t row = r0 + r < rows ? r0 + r : rows - 1;  // clamped rows compute a discarded result
        wr[r] = reinterpret_cast<const uint4 *>(w + row * cols);
    }
    float acc[ROWS][NT];
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[r][t] = 0.f;

    for (size_t c = lane; c < chunks; c += 64) {
        uint4 wv[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; ++r) wv[r] = ld_nt(wr[r] + c);
        float xf[NT][8];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (t < n) {
                const float4 *xp = reinterpret_cast<const float4 *>(x + (size_t)t * cols + c * 8);
                float4 a = xp[0], b = xp[1];
                xf[t][0] = a.x; xf[t][1] = a.y; xf[t][2] = a.z; xf[t][3] = a.w;
                xf[t][4] = b.x; xf[t][5] = b.y; xf[t][6] = b.z; xf[t][7] = b.w;
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) xf[t][i] = 0.f;
            }
        }
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            float wf[8];
            unpack8(wv[r], wf);
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[r][t] = fmaf(wf[i], xf[t][i], acc[r][t]);
        }
    }
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float s = wave_sum(acc[r][t]);
            if (lane == 0 && r0 + r < rows && t < n) out[(size_t)t * out_stride + r0 + r] = s;
        }
}

// Rows whose length is not a multiple of 8 (no 16-byte alignment): one wave
// per row, one element per lane per step.
__global__ __launch_bounds__(256) void gemv_scalar_kernel(float *__restrict__ out, const uint16_t *__restrict__ w,
                                                          size_t rows, size_t cols, const float *__restrict__ x,
                                                          size_t n) {
    const int lane = threadIdx.x & 63;
    const size_t r = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    for (size_t t = 0; t < n; ++t) {
        float acc = 0.f;
        for (size_t c = lane; c < cols; c += 64) acc = fmaf(bf16_to_f32(w[r * cols + c]), x[t * cols + c], acc);
        acc = wave_sum(acc);
        if (lane == 0) out[t * rows + r] = acc;
    }
}

template <int ROWS, int NT>
static hipError_t gemv(hipStream_t s, float *out, const uint16_t *w, size_t rows, size_t cols, const float *x,
                       int n, size_t out_stride) {
    size_t waves = (rows + ROWS - 1) / ROWS;
    unsigned blocks = (unsigned)((waves + 3) / 4);
    gemv_kernel<ROWS, NT><<<blocks, 256, 0, s>>>(out, w, rows, cols, x, n, out_stride);
    return hipGetLastError();
}

hipError_t launch_matmul(hipStream_t s, float *out, const uint16_t *w, size_t rows, size_t cols, const float *x,
                         size_t n) {
    if (n == 0 || rows == 0) return hipSuccess;
    if (cols % 8 != 0) {
        gemv_scalar_kernel<<<dim3((unsigned)((rows + 3) / 4)), 256, 0, s>>>(out, w, rows, cols, x, n);
        return hipGetLastError();
    }
    if (n >= kGemmMinTokens && gemm_supported(rows, cols)) return launch_gemm(s, out, w, rows, cols, x, n);
    if (n == 1) {
        // Enough waves to cover the chip (256 CUs x 4 SIMDs) before packing rows.
        if (rows >= 16384) return gemv<4, 1>(s, out, w, rows, cols, x, 1, rows);
        if (rows >= 4096) return gemv<2, 1>(s, out, w, rows, cols, x, 1, rows);
        return gemv<1, 1>(s, out, w, rows, cols, x, 1, rows);
    }
    for (size_t t0 = 0; t0 < n; t0 += 8) {
        int nt = (int)std::min<size_t>(8, n - t0);
        hipError_t e;
        if (nt <= 2) e = gemv<2, 2>(s, out + t0 * rows, w, rows, cols, x + t0 * cols, nt, rows);
        else if (nt <= 4) e = gemv<2, 4>(s, out + t0 * rows, w, rows, cols, x + t0 * cols, nt, rows);
        else e = gemv<2, 8>(s, out + t0 * rows, w, rows, cols, x + t0 * cols, nt, rows);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace th
