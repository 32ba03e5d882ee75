// bf16 MFMA GEMM for multi-token matmuls (prefill): out[t][r] = w[r] . x[t]
// (model/cpu.rs:49-77 for n tokens), on the gfx950 matrix cores.
//
// The weights are bf16 as uploaded; the activations are f32. Each activation
// is split into two bf16 terms, x = hi + lo with hi = bf16(x) and
// lo = bf16(x - hi), which together carry 16 significant bits (relative error
// <= 2^-17), and both are multiplied against the same weight fragment: two
// v_mfma_f32_16x16x32_bf16 per fragment pair, f32 accumulation. A plain bf16
// rounding of x would leave ~1e-3 relative error in every output.
//
// Tiling: a 256-thread block computes 64 tokens x 64 weight rows; each of its
// four waves a 32 x 32 quarter (2 x 2 MFMA tiles of 16 x 16). K advances 64 at
// a time through a ring of kStages LDS stages that the block fills with
// direct global->LDS loads (global_load_lds, 16 bytes a lane), kStages - 1
// steps ahead of the step being multiplied, so that a step's memory round trip
// overlaps the MFMAs of the steps before it. The activation tile stays f32 in
// LDS and is split into hi/lo while the A fragments are built.
//
// LDS rows are XOR-swizzled in 16-byte chunks so that the 16 rows one fragment
// read touches land on distinct banks: the DMA lane that writes physical chunk
// p of row r fetches logical chunk p ^ swizzle(r).
#include "gemm.h"

namespace th {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

constexpr int BM = 64, BN = 64, BK = 64;  // tokens, weight rows, columns per step
constexpr int NTHR = 256;
constexpr int kStages = 4;
constexpr int XCH = BK / 4;               // 16-byte chunks per activation row (f32)
constexpr int WCH = BK / 8;               // 16-byte chunks per weight row (bf16)
constexpr int X_CHUNKS = BM * XCH;        // 1024
constexpr int W_CHUNKS = BN * WCH;        // 512
constexpr int DMA_PER_WAVE = (X_CHUNKS + W_CHUNKS) / NTHR;  // 6 instructions per wave per step

struct alignas(16) Stage {
    uint4 x[X_CHUNKS];  // [BM][XCH] f32 rows, swizzled
    uint4 w[W_CHUNKS];  // [BN][WCH] bf16 rows, swizzled
};

__device__ __forceinline__ int x_swz(int row) { return row & (XCH - 1); }
__device__ __forceinline__ int w_swz(int row) { return (row >> 1) & (WCH - 1); }

__device__ __forceinline__ void dma16(const void *src, uint4 *lds_wave_base) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds_wave_base, 16, 0, 0);
}

// s_waitcnt vmcnt(N) leaving the other counters alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// Queues the loads of K step k0 into stage st: each wave fills whole 1 KB
// spans (64 lanes x 16 B) of the stage, four of the activation tile and two
// of the weight tile. Token rows past n read row n - 1 (their results are
// never stored).
__device__ __forceinline__ void issue_step(Stage &st, const float *x, const uint16_t *w, int t0, int r0, int n,
                                           int cols, int k0) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < X_CHUNKS / NTHR; ++i) {
        const int span = wave * (X_CHUNKS / NTHR) + i;
        const int p = span * 64 + lane, row = p / XCH, pc = p % XCH;
        const int t = min(t0 + row, n - 1);
        dma16(x + (size_t)t * cols + k0 + (pc ^ x_swz(row)) * 4, st.x + span * 64);
    }
#pragma unroll
    for (int i = 0; i < W_CHUNKS / NTHR; ++i) {
        const int span = wave * (W_CHUNKS / NTHR) + i;
        const int p = span * 64 + lane, row = p / WCH, pc = p % WCH;
        dma16(w + (size_t)(r0 + row) * cols + k0 + (pc ^ w_swz(row)) * 8, st.w + span * 64);
    }
}

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
}

// A fragments (hi, lo) of token row `row`, columns 8 (lane / 16) + kb .. + 8.
__device__ __forceinline__ void a_frag(const Stage &st, int row, int lc, bf16x8 &hi, bf16x8 &lo) {
    const uint4 c0 = st.x[row * XCH + (lc ^ x_swz(row))];
    const uint4 c1 = st.x[row * XCH + ((lc + 1) ^ x_swz(row))];
    const float v[8] = {__uint_as_float(c0.x), __uint_as_float(c0.y), __uint_as_float(c0.z), __uint_as_float(c0.w),
                        __uint_as_float(c1.x), __uint_as_float(c1.y), __uint_as_float(c1.z), __uint_as_float(c1.w)};
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h[i] = pack_bf16(v[2 * i], v[2 * i + 1]);
        l[i] = pack_bf16(v[2 * i] - __uint_as_float(h[i] << 16), v[2 * i + 1] - __uint_as_float(h[i] & 0xffff0000u));
    }
    hi = __builtin_bit_cast(bf16x8, make_uint4(h[0], h[1], h[2], h[3]));
    lo = __builtin_bit_cast(bf16x8, make_uint4(l[0], l[1], l[2], l[3]));
}

__device__ __forceinline__ bf16x8 b_frag(const Stage &st, int row, int lc) {
    return __builtin_bit_cast(bf16x8, st.w[row * WCH + (lc ^ w_swz(row))]);
}

__global__ __launch_bounds__(NTHR) void gemm_kernel(float *__restrict__ out, const uint16_t *__restrict__ w,
                                                    const float *__restrict__ x, int n, int rows, int cols) {
    __shared__ Stage ring[kStages];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t0 = blockIdx.y * BM, r0 = blockIdx.x * BN;
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    const int fr = lane & 15, fq = lane >> 4;  // fragment row, quarter of the K slice
    const int nk = cols / BK;

    f32x4 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int s = 0; s < kStages - 1; ++s)
        if (s < nk) issue_step(ring[s], x, w, t0, r0, n, cols, s * BK);

    for (int k = 0; k < nk; ++k) {
        // This wave's loads of step k are done once at most the later steps'
        // loads are outstanding; the barrier makes every wave's visible and
        // frees the stage step k - 1 used.
        if (k + kStages - 2 < nk) wait_vm<(kStages - 2) * DMA_PER_WAVE>();
        else wait_vm<0>();
        __syncthreads();
        if (k + kStages - 1 < nk) issue_step(ring[(k + kStages - 1) % kStages], x, w, t0, r0, n, cols,
                                             (k + kStages - 1) * BK);
        const Stage &st = ring[k % kStages];
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            bf16x8 ah[2], al[2], b[2];
#pragma unroll
            for (int m = 0; m < 2; ++m) a_frag(st, wm + m * 16 + fr, ks * 8 + fq * 2, ah[m], al[m]);
#pragma unroll
            for (int q = 0; q < 2; ++q) b[q] = b_frag(st, wn + q * 16 + fr, ks * 4 + fq);
#pragma unroll
            for (int m = 0; m < 2; ++m)
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    acc[m][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[m], b[q], acc[m][q], 0, 0, 0);
                    acc[m][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[m], b[q], acc[m][q], 0, 0, 0);
                }
        }
    }
    // D[4 (l / 16) + i][l % 16]: token rows, weight-row columns.
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = t0 + wm + m * 16 + fq * 4 + i;
                if (t < n) out[(size_t)t * rows + r0 + wn + q * 16 + fr] = acc[m][q][i];
            }
}

}  // namespace

bool gemm_supported(size_t rows, size_t cols) {
    return rows % BN == 0 && cols % BK == 0 && rows / BN <= 65535 && rows * cols < ((size_t)1 << 40) &&
           cols < ((size_t)1 << 30);
}

hipError_t launch_gemm(hipStream_t s, float *out, const uint16_t *w, size_t rows, size_t cols, const float *x,
                       size_t n) {
    if (n == 0 || rows == 0) return hipSuccess;
    if (!gemm_supported(rows, cols) || (n + BM - 1) / BM > 65535 || n > ((size_t)1 << 30)) return hipErrorInvalidValue;
    static_assert(sizeof(Stage) * kStages <= 160 * 1024, "LDS ring exceeds the CU's LDS");
    dim3 grid((unsigned)(rows / BN), (unsigned)((n + BM - 1) / BM));
    gemm_kernel<<<grid, NTHR, 0, s>>>(out, w, x, (int)n, (int)rows, (int)cols);
    return hipGetLastError();
}

}  // namespace th
