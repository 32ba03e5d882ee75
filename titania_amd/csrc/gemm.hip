// bf16 MFMA GEMM for multi-token matmuls (prefill): out[t][r] = w[r] . x[t]
// (model/cpu.rs:49-77 for n tokens), on the gfx950 matrix cores.
//
// The weights are bf16 as uploaded; the activations are f32. A first kernel
// splits every activation into two bf16 terms, x = hi + lo with hi = bf16(x)
// and lo = bf16(x - hi), which together carry 16 significant bits (relative
// error <= 2^-17); the GEMM multiplies both against the same weight fragment
// (two v_mfma_f32_16x16x32_bf16 per fragment pair, f32 accumulation). A plain
// bf16 rounding of x would leave ~1e-3 relative error in every output.
//
// Tiling: a 256-thread block computes 64 tokens x 64 weight rows; each of its
// four waves a 32 x 32 quarter (2 x 2 MFMA tiles of 16 x 16). K advances 64 at
// a time through a ring of kStages LDS stages (hi, lo and weight tiles, 24 KB
// each, so two blocks fit a CU) that the block fills with direct global->LDS
// loads (global_load_lds, 16 bytes a lane) kStages - 1 steps ahead of the step
// being multiplied. Rows of every tile are XOR-swizzled in 16-byte chunks so
// that the 16 rows a fragment read touches land on distinct banks: the lane
// that writes physical chunk p of row r fetches logical chunk p ^ swizzle(r).
// One launch may cover several weight matrices that share the input (q, k and
// v; gate and up): their rows are concatenated.
#include "gemm.h"

#include "device_util.h"

namespace th {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

constexpr int BM = 64, BN = 64, BK = 64;  // tokens, weight rows, columns per step
constexpr int NTHR = 256;
constexpr int kStages = 3;
constexpr int CH = BK / 8;                // 16-byte chunks per tile row (bf16)
constexpr int TILE = BM * CH;             // 512 chunks per tile
constexpr int DMA_PER_WAVE = 3 * TILE / NTHR;  // 6 instructions per wave per step

struct alignas(16) Stage {
    uint4 hi[TILE], lo[TILE];  // [BM][CH] activation halves
    uint4 w[TILE];             // [BN][CH] weights
};

__device__ __forceinline__ int swz(int row) { return (row >> 1) & (CH - 1); }

__device__ __forceinline__ void dma16(const void *src, uint4 *lds_wave_base) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds_wave_base, 16, 0, 0);
}

// s_waitcnt vmcnt(N) leaving the other counters alone (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// Up to three weight matrices of `cols` columns, rows concatenated.
struct Segs {
    const uint16_t *w[3];
    float *out[3];
    int rows[3];
    int n;
};

// The row tile r0 (a multiple of BN) of the concatenation: its matrix and local row.
__device__ __forceinline__ int seg_of(const Segs &s, int r0, int &local) {
    if (r0 < s.rows[0]) {
        local = r0;
        return 0;
    }
    if (r0 < s.rows[0] + s.rows[1]) {
        local = r0 - s.rows[0];
        return 1;
    }
    local = r0 - s.rows[0] - s.rows[1];
    return 2;
}

// Queues the loads of K step k0 into stage st: each wave fills whole 1 KB
// spans (64 lanes x 16 B) of the stage, two of each tile. Token rows past n
// read row n - 1 (their results are never stored).
__device__ __forceinline__ void issue_step(Stage &st, const uint16_t *hi, const uint16_t *lo, const uint16_t *w,
                                           int t0, int n, int cols, int k0) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < TILE / NTHR; ++i) {
        const int span = wave * (TILE / NTHR) + i;
        const int p = span * 64 + lane, row = p / CH, pc = p % CH;
        const int t = min(t0 + row, n - 1);
        const size_t off = (size_t)t * cols + k0 + (pc ^ swz(row)) * 8;
        dma16(hi + off, st.hi + span * 64);
        dma16(lo + off, st.lo + span * 64);
        dma16(w + (size_t)row * cols + k0 + (pc ^ swz(row)) * 8, st.w + span * 64);
    }
}

__device__ __forceinline__ bf16x8 frag(const uint4 *tile, int row, int lc) {
    return __builtin_bit_cast(bf16x8, tile[row * CH + (lc ^ swz(row))]);
}

// With ksplit > 1 (one matrix), block z of the grid's third dimension takes
// K steps [z nk / ksplit, (z + 1) nk / ksplit) and stores its partial tile in
// part[z][t][r]; launch_gemm_multi then sums the partials in z order.
__global__ __launch_bounds__(NTHR, 2) void gemm_kernel(Segs sg, const uint16_t *__restrict__ hi,
                                                        const uint16_t *__restrict__ lo, int n, int cols,
                                                        float *__restrict__ part, int ksplit) {
    __shared__ Stage ring[kStages];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t0 = blockIdx.y * BM;
    int rl;
    const int sgi = seg_of(sg, blockIdx.x * BN, rl);
    const int wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
    const int fr = lane & 15, fq = lane >> 4;  // fragment row, quarter of the K slice
    const int nk_all = cols / BK, z = blockIdx.z;
    const int kb = (int)((long long)z * nk_all / ksplit), nk = (int)((long long)(z + 1) * nk_all / ksplit) - kb;
    const uint16_t *w = sg.w[sgi] + (size_t)rl * cols + (size_t)kb * BK;
    hi += (size_t)kb * BK;
    lo += (size_t)kb * BK;

    f32x4 acc[2][2];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int b = 0; b < 2; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int s = 0; s < kStages - 1; ++s)
        if (s < nk) issue_step(ring[s], hi, lo, w, t0, n, cols, s * BK);

    for (int k = 0; k < nk; ++k) {
        // This wave's loads of step k are done once at most the later steps'
        // loads are outstanding; the barrier makes every wave's visible and
        // frees the stage step k - 1 used.
        if (k + kStages - 2 < nk) wait_vm<(kStages - 2) * DMA_PER_WAVE>();
        else wait_vm<0>();
        __syncthreads();
        if (k + kStages - 1 < nk)
            issue_step(ring[(k + kStages - 1) % kStages], hi, lo, w, t0, n, cols, (k + kStages - 1) * BK);
        const Stage &st = ring[k % kStages];
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            const int lc = ks * 4 + fq;
            bf16x8 ah[2], al[2], b[2];
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                ah[m] = frag(st.hi, wm + m * 16 + fr, lc);
                al[m] = frag(st.lo, wm + m * 16 + fr, lc);
            }
#pragma unroll
            for (int q = 0; q < 2; ++q) b[q] = frag(st.w, wn + q * 16 + fr, lc);
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
    const int rows = sg.rows[sgi];
    float *out = ksplit > 1 ? part + (size_t)z * n * rows : sg.out[sgi];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = t0 + wm + m * 16 + fq * 4 + i;
                if (t < n) out[(size_t)t * rows + rl + wn + q * 16 + fr] = acc[m][q][i];
            }
}

// split_bf16 of 4 elements a thread.
__global__ void split_kernel(const float4 *__restrict__ x, uint2 *__restrict__ hi, uint2 *__restrict__ lo, size_t n4) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) split_bf16x4(x[i], hi[i], lo[i]);
}

// out[i] = sum over z < ksplit of part[z * m + i] (z in order), 4 a thread.
__global__ void splitk_sum_kernel(const float4 *__restrict__ part, float4 *__restrict__ out, size_t m4, int ksplit) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < m4; i += stride) {
        float4 acc = part[i];
        for (int z = 1; z < ksplit; ++z) {
            const float4 v = part[(size_t)z * m4 + i];
            acc.x += v.x;
            acc.y += v.y;
            acc.z += v.z;
            acc.w += v.w;
        }
        out[i] = acc;
    }
}

}  // namespace

bool gemm_supported(size_t rows, size_t cols) {
    return rows % BN == 0 && cols % BK == 0 && rows < ((size_t)1 << 24) && cols < ((size_t)1 << 20) &&
           rows * cols < ((size_t)1 << 40);
}

size_t gemm_scratch_bytes(size_t n, size_t cols, size_t rows) {
    return n * cols * 2 * sizeof(uint16_t) + (size_t)kGemmMaxSplitK * n * rows * sizeof(float);
}

hipError_t launch_gemm_split(hipStream_t s, const float *x, size_t n, size_t cols, uint16_t *hi, uint16_t *lo) {
    if (n == 0) return hipSuccess;
    if (cols % 4 || !x || !hi || !lo) return hipErrorInvalidValue;
    const size_t n4 = n * cols / 4;
    const unsigned blocks = (unsigned)std::min<size_t>((n4 + 255) / 256, 4096);
    split_kernel<<<blocks, 256, 0, s>>>(reinterpret_cast<const float4 *>(x), reinterpret_cast<uint2 *>(hi),
                                        reinterpret_cast<uint2 *>(lo), n4);
    return hipGetLastError();
}

// A single matrix with few output tiles (o, down: 1024 rows) splits K so that
// the launch still fills the chip, keeping at least 4 K steps per split.
int gemm_ksplit(size_t n, size_t rows, size_t cols, int n_outs) {
    if (n_outs != 1) return 1;
    const size_t tiles = (rows / BN) * ((n + BM - 1) / BM), nk = cols / BK;
    int ksplit = 1;
    while (ksplit < kGemmMaxSplitK && tiles * ksplit < 512 && (size_t)ksplit * 2 * 4 <= nk) ksplit *= 2;
    return ksplit;
}

hipError_t launch_gemm_hl(hipStream_t s, const uint16_t *hi, const uint16_t *lo, size_t n, size_t cols,
                          const GemmOut *outs, int n_outs, float *part, int ksplit) {
    if (n == 0) return hipSuccess;
    if (n_outs < 1 || n_outs > 3 || !hi || !lo || (n + BM - 1) / BM > 65535 || n > ((size_t)1 << 24) ||
        ksplit < 1 || ksplit > kGemmMaxSplitK || (ksplit > 1 && (n_outs != 1 || !part)) ||
        (size_t)ksplit > cols / BK)
        return hipErrorInvalidValue;
    Segs sg{};
    size_t total = 0;
    for (int i = 0; i < n_outs; ++i) {
        if (!gemm_supported(outs[i].rows, cols)) return hipErrorInvalidValue;
        sg.w[i] = outs[i].w;
        sg.out[i] = outs[i].out;
        sg.rows[i] = (int)outs[i].rows;
        total += outs[i].rows;
    }
    sg.n = n_outs;
    if (total / BN > 65535) return hipErrorInvalidValue;
    dim3 grid((unsigned)(total / BN), (unsigned)((n + BM - 1) / BM), (unsigned)ksplit);
    gemm_kernel<<<grid, NTHR, 0, s>>>(sg, hi, lo, (int)n, (int)cols, part, ksplit);
    return hipGetLastError();
}

hipError_t launch_gemm_multi(hipStream_t s, const float *x, size_t n, size_t cols, const GemmOut *outs, int n_outs,
                             void *scratch, size_t scratch_bytes) {
    if (n == 0) return hipSuccess;
    if (n_outs < 1 || n_outs > 3 || !scratch || n * cols * 2 * sizeof(uint16_t) > scratch_bytes)
        return hipErrorInvalidValue;
    size_t total = 0;
    for (int i = 0; i < n_outs; ++i) total += outs[i].rows;
    uint16_t *hi = static_cast<uint16_t *>(scratch), *lo = hi + n * cols;
    float *part = reinterpret_cast<float *>(hi + 2 * n * cols);
    // The partial tiles take the rest of the scratch; fewer splits when it is short.
    int ksplit = gemm_ksplit(n, total, cols, n_outs);
    while (ksplit > 1 && n * cols * 4 + (size_t)ksplit * n * total * sizeof(float) > scratch_bytes) ksplit /= 2;
    hipError_t e = launch_gemm_split(s, x, n, cols, hi, lo);
    if (e == hipSuccess) e = launch_gemm_hl(s, hi, lo, n, cols, outs, n_outs, part, ksplit);
    if (e != hipSuccess || ksplit == 1) return e;
    const size_t m4 = n * total / 4;
    splitk_sum_kernel<<<(unsigned)std::min<size_t>((m4 + 255) / 256, 4096), 256, 0, s>>>(
        reinterpret_cast<const float4 *>(part), reinterpret_cast<float4 *>(outs[0].out), m4, ksplit);
    return hipGetLastError();
}

hipError_t launch_gemm(hipStream_t s, float *out, const uint16_t *w, size_t rows, size_t cols, const float *x,
                       size_t n) {
    if (n == 0 || rows == 0) return hipSuccess;
    if (!gemm_supported(rows, cols)) return hipErrorInvalidValue;
    // The split activations live in stream-ordered scratch for this call.
    void *scratch = nullptr;
    const size_t bytes = gemm_scratch_bytes(n, cols, rows);
    hipError_t e = hipMallocAsync(&scratch, bytes, s);
    if (e != hipSuccess) return e;
    const GemmOut o{w, rows, out};
    e = launch_gemm_multi(s, x, n, cols, &o, 1, scratch, bytes);
    const hipError_t f = hipFreeAsync(scratch, s);
    return e != hipSuccess ? e : f;
}

}  // namespace th
