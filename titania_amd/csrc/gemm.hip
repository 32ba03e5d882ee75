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
// Tiling: a 256-thread block computes 64 tokens x 64 weight rows (the small
// tile; each of its four waves a 32 x 32 quarter, 2 x 2 MFMA tiles of 16 x 16)
// or, in launches of many tiles, a 512-thread block 128 x 128 (the large
// tile; eight waves of 32 tokens x 64 rows, 2 x 4 MFMA tiles, two waves a
// SIMD). K advances 64 at a time through a ring of 3 LDS stages (hi, lo and
// weight tiles: 24 KB a stage for the small tile, so two blocks fit a CU;
// 48 KB for the large tile, one block a CU) that the block fills with direct
// global->LDS loads (global_load_lds, 16 bytes a lane) two steps ahead of the
// step being multiplied. Rows of every tile are XOR-swizzled in 16-byte chunks so
// that the 16 rows a fragment read touches land on distinct banks: the lane
// that writes physical chunk p of row r fetches logical chunk p ^ swizzle(r).
// One launch may cover several weight matrices that share the input (q, k and
// v; gate and up): their rows are concatenated.
#include "gemm.h"

#include "device_util.h"
#include "fused.h"

namespace th {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

constexpr int BK = 64;                    // K range multiple every launch needs

// A block tile of BM tokens x BN weight rows, its WGM x WGN waves each a
// BM/WGM x BN/WGN part, K staged BK columns at a time through `STAGES` LDS
// stages.
template <int BM_, int BN_, int BK_, int STAGES_, int WGM_ = 2, int WGN_ = 2, bool REG_PAIRS_ = false>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, kStages = STAGES_;
    // Paired (gate/up) tiles: the weight tile interleaves 16-row groups of
    // gate and up, so that a wave holds both halves of its outputs and the
    // SiLU epilogue runs in registers (otherwise they meet in LDS).
    static constexpr bool REG_PAIRS = REG_PAIRS_;
    static constexpr int WGM = WGM_, WGN = WGN_, NT = 64 * WGM * WGN;  // waves: WGM down x WGN across
    static constexpr int CH = BK / 8;  // 16-byte chunks per tile row (bf16)
    static constexpr int TA = BM * CH, TB = BN * CH;     // 16-byte chunks per tile
    static constexpr int FM = BM / WGM / 16, FN = BN / WGN / 16;  // 16 x 16 fragments per wave
    static constexpr int DMA_PER_WAVE = (2 * TA + TB) / NT;
    // issue_step deals whole 64-lane spans of each tile to the waves.
    static_assert(TA % NT == 0 && TB % NT == 0, "every wave loads the same whole spans of each tile");
    struct alignas(16) Stage {
        uint4 hi[TA], lo[TA];  // [BM][CH] activation halves
        uint4 w[TB];           // [BN][CH] weights
    };
};
using Small = Tile<64, 64, 64, 3>;    // 24 KB a stage: two blocks a CU
// The small tile with two stages (48 KB): three blocks a CU. For the gate/up
// GEMM of launches with more small tiles than two a CU, where the rounds of
// blocks matter more than the deeper ring (Qwen3-0.6B prefill, paired runs:
// 512 tokens, 768 tiles, 2.89-2.94 -> 2.86-2.92 ms; 1024 tokens 4.88-4.90 ->
// 4.81-4.82 ms).
using Small2 = Tile<64, 64, 64, 2>;
using Large = Tile<128, 128, 64, 3, 4, 2>;  // 48 KB a stage: one block a CU, eight waves of 32 x 64
using Head = Tile<32, 128, 64, 3>;          // one attention head's 128 rows: 24 KB a stage, two blocks a CU
// 48 KB a stage of 32 K columns: one block a CU, eight waves of 64 x 128. A
// wave reads 16 fragments from LDS per 64 products, against 8 per 16 in the
// 32 x 64 waves of the large tile.
using Huge = Tile<256, 256, 32, 3, 4, 2, true>;

// The XOR swizzle of a row's 16-byte chunks: a fragment read takes one chunk
// of 16 consecutive rows, and the 64 banks span 256 bytes, 16 / CH rows of
// CH chunks; rows that share a bank span differ in the swizzle.
template <int CH>
__device__ __forceinline__ int swz(int row) { return (row / (16 / CH)) & (CH - 1); }

// The block barrier of the K loop. __syncthreads() would also wait for every
// load still in flight (its workgroup fence covers the LDS writes of
// global_load_lds, even with the fence narrowed to LDS), the later stages'
// too, leaving one step of the ring in flight instead of two. Each wave has
// already waited for its own loads of the step about to be read (vmcnt counts
// a global_load_lds until its LDS write is done) and has consumed its reads
// of the stage about to be refilled (its MFMAs used them), so the hardware
// barrier alone orders both; the signal fences keep the compiler from moving
// memory accesses across it.
__device__ __forceinline__ void stage_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Up to three weight matrices of `cols` columns, rows concatenated.
struct Segs {
    const uint16_t *w[3];
    float *out[3];
    int rows[3];
    int n;
};

// Queues the loads of K step k0 into stage st: each wave fills whole 1 KB
// spans (64 lanes x 16 B) of the stage. Weight rows [0, BN/2) of the tile
// come from wa, the rest from wb (with IL, 16-row groups alternate between
// them). Token rows past n read row n - 1 (their results are never stored).
template <class T, bool IL = false>
__device__ __forceinline__ void issue_step(typename T::Stage &st, const uint16_t *hi, const uint16_t *lo,
                                           const uint16_t *wa, const uint16_t *wb, int t0, int n, int cols,
                                           int k0) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    auto w_row = [&](int row) {
        if constexpr (IL)  // 16-row groups alternate between wa and wb
            return ((row >> 4) & 1 ? wb : wa) + (size_t)((row >> 5) * 16 + (row & 15)) * cols;
        return row < T::BN / 2 ? wa + (size_t)row * cols : wb + (size_t)(row - T::BN / 2) * cols;
    };
    if constexpr (T::TA == T::TB) {
#pragma unroll
        for (int i = 0; i < T::TA / T::NT; ++i) {
            const int span = wave * (T::TA / T::NT) + i;
            const int p = span * 64 + lane, row = p / T::CH, pc = p % T::CH;
            const int t = min(t0 + row, n - 1);
            const size_t off = (size_t)t * cols + k0 + (pc ^ swz<T::CH>(row)) * 8;
            dma16(hi + off, st.hi + span * 64);
            dma16(lo + off, st.lo + span * 64);
            dma16(w_row(row) + k0 + (pc ^ swz<T::CH>(row)) * 8, st.w + span * 64);
        }
    } else {
#pragma unroll
        for (int i = 0; i < T::TA / T::NT; ++i) {
            const int span = wave * (T::TA / T::NT) + i;
            const int p = span * 64 + lane, row = p / T::CH, pc = p % T::CH;
            const int t = min(t0 + row, n - 1);
            const size_t off = (size_t)t * cols + k0 + (pc ^ swz<T::CH>(row)) * 8;
            dma16(hi + off, st.hi + span * 64);
            dma16(lo + off, st.lo + span * 64);
        }
#pragma unroll
        for (int i = 0; i < T::TB / T::NT; ++i) {
            const int span = wave * (T::TB / T::NT) + i;
            const int p = span * 64 + lane, row = p / T::CH, pc = p % T::CH;
            dma16(w_row(row) + k0 + (pc ^ swz<T::CH>(row)) * 8, st.w + span * 64);
        }
    }
}

template <int CH>
__device__ __forceinline__ bf16x8 frag(const uint4 *tile, int row, int lc) {
    return __builtin_bit_cast(bf16x8, tile[row * CH + (lc ^ swz<CH>(row))]);
}

// The (column tile, row tile) of this block. Blocks are dealt to the 8 XCDs
// in turn (linear block id mod 8), and the blocks that one XCD runs at once
// share its L2. In launch order, 32 consecutive blocks would otherwise take
// 32 different weight tiles of one row of tokens, so every weight chunk would
// miss in L2. Here each XCD takes a contiguous range of tiles, ordered in
// panels of PANEL row tiles (down the panel, then across): the blocks an XCD
// runs together cover a few weight tiles and a few token tiles, and share
// both. The map is a bijection whatever the XCD count; only the speed assumes it.
// gx, gy: the grid's x and y sizes, passed by the kernels as leading
// arguments (preloaded into SGPRs with the others; the grid's size is
// otherwise one more fetch before a block's first loads can be addressed).
template <int PANEL>
__device__ __forceinline__ void tile_of_block(int &tx, int &ty, int gx, int gy) {
    const int nt = gx * gy;
    const int lin = (int)blockIdx.x + (int)blockIdx.y * gx;
    constexpr int kXcds = 8;
    const int xcd = lin % kXcds, i = lin / kXcds, q = nt / kXcds, r = nt % kXcds;
    const int t = xcd * q + (xcd < r ? xcd : r) + i;  // this XCD's range starts at xcd q + min(xcd, r)
    const int ph = gy < PANEL ? gy : PANEL;           // rows of a full panel
    const int panel = t / (ph * gx), w = t % (ph * gx);
    const int rows = gy - panel * ph < ph ? gy - panel * ph : ph;  // rows of this (maybe last) panel
    tx = w / rows;
    ty = panel * ph + w % rows;
}

// The matrix that the row tile r0 of the concatenation falls in: its weights
// from its local row, output, row count and local row. Selected without
// indexing the argument arrays by a run-time value, which would copy them to
// scratch memory.
struct SegTile {
    const uint16_t *w;
    float *out;
    int rows, local;
};

// A paired tile (SiLU epilogue): weight rows [r0, r0 + BN/2) of gate and of
// up, and the h = silu(gate) * up output as hi/lo terms [n][inter].
struct PairTile {
    const uint16_t *gate, *up;
    uint16_t *h_hi, *h_lo;
    int inter, r0;
};

__device__ __forceinline__ SegTile seg_tile(const uint16_t *w0, float *out0, int n0, const Segs &s, int r0) {
    const int n1 = s.rows[1];
    if (r0 < n0) return SegTile{w0, out0, n0, r0};
    if (r0 < n0 + n1) return SegTile{s.w[1], s.out[1], n1, r0 - n0};
    return SegTile{s.w[2], s.out[2], s.rows[2], r0 - n0 - n1};
}

// With ksplit > 1 (one matrix), block z of the grid's third dimension takes
// K steps [z nk / ksplit, (z + 1) nk / ksplit) and stores its partial tile in
// part[z][t][r]; the consumer sums the partials in z order.
// Epilogues: store the tile (or its split-K partial), SiLU * up of paired
// gate/up rows, or the q/k/v post-processing of one attention head.
enum Epi { kStoreTile, kSiluPairs, kQkvHead, kQkvHeads };

// The head of a q/k/v head tile: role 0 q, 1 k, 2 v; index within the role.
struct HeadTile {
    const QkvPostArgs *a;
    int role, head;
};

template <class T, int EPI = kStoreTile, typename KV = float>
__device__ __forceinline__ void gemm_tile(int ty, SegTile sg, const uint16_t *__restrict__ hi,
                                          const uint16_t *__restrict__ lo, int n, int cols,
                                          float *__restrict__ part, int ksplit, PairTile pt = {},
                                          HeadTile ht = {}) {
    constexpr bool PAIRED = EPI == kSiluPairs;
    constexpr bool IL = PAIRED && T::REG_PAIRS;
    constexpr int FM = T::FM, FN = T::FN, kStages = T::kStages;
    __shared__ typename T::Stage ring[kStages];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int t0 = ty * T::BM;
    const int rl = sg.local;
    const int wm = (wave / T::WGN) * (T::BM / T::WGM), wn = (wave % T::WGN) * (T::BN / T::WGN);
    const int fr = lane & 15, fq = lane >> 4;  // fragment row, quarter of the K slice
    const int nk_all = cols / T::BK, z = blockIdx.z;
    const int kb = (int)((long long)z * nk_all / ksplit), nk = (int)((long long)(z + 1) * nk_all / ksplit) - kb;
    const uint16_t *wa = PAIRED ? pt.gate + (size_t)pt.r0 * cols + (size_t)kb * T::BK
                                : sg.w + (size_t)rl * cols + (size_t)kb * T::BK;
    const uint16_t *wb = PAIRED ? pt.up + (size_t)pt.r0 * cols + (size_t)kb * T::BK
                                : wa + (size_t)(T::BN / 2) * cols;
    (void)ht;
    hi += (size_t)kb * T::BK;
    lo += (size_t)kb * T::BK;

    f32x4 acc[FM][FN];
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
    for (int s = 0; s < kStages - 1; ++s)
        if (s < nk) issue_step<T, IL>(ring[s], hi, lo, wa, wb, t0, n, cols, s * T::BK);

    for (int k = 0; k < nk; ++k) {
        // This wave's loads of step k are done once at most the later steps'
        // loads are outstanding; the barrier makes every wave's visible and
        // frees the stage step k - 1 used.
        if (k + kStages - 2 < nk) wait_vm<(kStages - 2) * T::DMA_PER_WAVE>();
        else wait_vm<0>();
        stage_barrier();
        const typename T::Stage &st = ring[k % kStages];
#pragma unroll
        for (int ks = 0; ks < T::BK / 32; ++ks) {
            const int lc = ks * 4 + fq;
            bf16x8 ah[FM], al[FM], b[FN];
#pragma unroll
            for (int m = 0; m < FM; ++m) {
                ah[m] = frag<T::CH>(st.hi, wm + m * 16 + fr, lc);
                al[m] = frag<T::CH>(st.lo, wm + m * 16 + fr, lc);
            }
#pragma unroll
            for (int q = 0; q < FN; ++q) b[q] = frag<T::CH>(st.w, wn + q * 16 + fr, lc);
            // The next stage's loads go out while these fragment reads are in
            // flight: the address arithmetic of the DMA no longer sits between
            // the barrier and the first MFMA (4B 8192-token prefill 156.2 ->
            // 153.8 ms in a paired run).
            if (ks == 0 && k + kStages - 1 < nk)
                issue_step<T, IL>(ring[(k + kStages - 1) % kStages], hi, lo, wa, wb, t0, n, cols,
                                  (k + kStages - 1) * T::BK);
#pragma unroll
            for (int m = 0; m < FM; ++m)
#pragma unroll
                for (int q = 0; q < FN; ++q) {
                    acc[m][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[m], b[q], acc[m][q], 0, 0, 0);
                    acc[m][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[m], b[q], acc[m][q], 0, 0, 0);
                }
        }
    }
    // D[4 (l / 16) + i][l % 16]: token rows, weight-row columns.
    if constexpr (IL) {
        // Fragments 2p and 2p + 1 of a wave hold gate and up of the same 16
        // outputs: h = silu(g) * u straight from the accumulators.
        static_assert(FN % 2 == 0 && (T::BN / T::WGN) % 32 == 0, "whole gate/up fragment pairs a wave");
#pragma unroll
        for (int m = 0; m < FM; ++m)
#pragma unroll
            for (int p = 0; p < FN / 2; ++p)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = t0 + wm + m * 16 + fq * 4 + i;
                    if (t >= n) continue;
                    uint16_t h, l;
                    split_bf16(silu(acc[m][2 * p][i]) * acc[m][2 * p + 1][i], h, l);
                    const size_t o = (size_t)t * pt.inter + pt.r0 + wn / 2 + p * 16 + fr;
                    pt.h_hi[o] = h;
                    pt.h_lo[o] = l;
                }
        return;
    } else if constexpr (PAIRED) {
        // gate and up of a row sit in different waves: through LDS (the ring
        // is free once every wave has left the K loop), then h = silu(g) * u
        // as hi/lo terms, four outputs a thread.
        constexpr int EPS = T::BN + 4, HALF = T::BN / 2;
        static_assert(sizeof(ring) >= sizeof(float) * T::BM * EPS, "the epilogue tile fits the ring");
        float *ep = reinterpret_cast<float *>(ring);
        __syncthreads();
#pragma unroll
        for (int m = 0; m < FM; ++m)
#pragma unroll
            for (int q = 0; q < FN; ++q)
#pragma unroll
                for (int i = 0; i < 4; ++i) ep[(wm + m * 16 + fq * 4 + i) * EPS + wn + q * 16 + fr] = acc[m][q][i];
        __syncthreads();
        for (int e = tid; e < T::BM * HALF / 4; e += T::NT) {
            const int row = e / (HALF / 4), c = 4 * (e % (HALF / 4));
            if (t0 + row >= n) continue;
            const float4 g = *reinterpret_cast<const float4 *>(ep + row * EPS + c);
            const float4 u = *reinterpret_cast<const float4 *>(ep + row * EPS + HALF + c);
            uint2 h, l;
            split_bf16x4(make_float4(silu(g.x) * u.x, silu(g.y) * u.y, silu(g.z) * u.z, silu(g.w) * u.w), h, l);
            const size_t o = (size_t)(t0 + row) * pt.inter + pt.r0 + c;
            *reinterpret_cast<uint2 *>(pt.h_hi + o) = h;
            *reinterpret_cast<uint2 *>(pt.h_lo + o) = l;
        }
        return;
    }
    if constexpr (EPI == kQkvHeads) {
        // Waves of 64 tokens x 128 rows: one attention head each, whose
        // post-processing runs in registers. Lane (fq, fr) holds, for each of
        // its 16 tokens m 16 + 4 fq + i, dimensions 16 q + fr (q < 8): the
        // RMSNorm's sum of squares adds its 8 and then the 16 lanes of the
        // token (an xor butterfly, which leaves the same sum in every lane),
        // and the RoPE pairs (d, d + 64) are registers q and q + 4.
        static_assert(T::BN / T::WGN == 128 && FN == 8, "one head of 128 dimensions a wave");
        const QkvPostArgs &a = *ht.a;
        const long long pos0 = a.pos_dev ? *a.pos_dev : a.pos;
        const int head = ht.head + wn / 128;
        if (ht.role < 2) {
            const uint16_t *gain = ht.role == 0 ? a.q_norm : a.k_norm;
            float gv[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) gv[q] = gain ? bf16_to_f32(gain[q * 16 + fr]) : 1.f;
#pragma unroll
            for (int m = 0; m < FM; ++m)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = t0 + wm + m * 16 + fq * 4 + i;
                    const long long pos = pos0 + (t < n ? t : n - 1);
                    float x[8];
#pragma unroll
                    for (int q = 0; q < 8; ++q) x[q] = acc[m][q][i];
                    if (gain) {
                        float ss = 0.f;
#pragma unroll
                        for (int q = 0; q < 8; ++q) ss += x[q] * x[q];
                        ss += __shfl_xor(ss, 1, 16);
                        ss += __shfl_xor(ss, 2, 16);
                        ss += __shfl_xor(ss, 4, 16);
                        ss += __shfl_xor(ss, 8, 16);
                        const float scale = 1.0f / sqrtf(ss / 128.f + a.eps);
#pragma unroll
                        for (int q = 0; q < 8; ++q) x[q] = x[q] * (scale * gv[q]);
                    }
                    const float2 *ang = reinterpret_cast<const float2 *>(a.rope + pos * 128);
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float2 cs = ang[q * 16 + fr];
                        const float x0 = x[q] * cs.x - x[q + 4] * cs.y;
                        const float x1 = x[q + 4] * cs.x + x[q] * cs.y;
                        x[q] = x0;
                        x[q + 4] = x1;
                    }
                    if (t >= n) continue;
                    if (ht.role == 0) {
                        float *dst = a.q + ((long long)t * a.n_heads + head) * 128;
#pragma unroll
                        for (int q = 0; q < 8; ++q) dst[q * 16 + fr] = x[q];
                    } else {
                        KV *kc = reinterpret_cast<KV *>(a.k_cache) + (long long)head * a.head_stride +
                                 pos * a.pos_stride;
#pragma unroll
                        for (int q = 0; q < 8; ++q) store_kv(kc + q * 16 + fr, x[q]);
                        if (a.kh) {
                            const long long o = ((long long)head * a.plane_len + pos) * 128;
#pragma unroll
                            for (int q = 0; q < 8; ++q) split_bf16(x[q], a.kh[o + q * 16 + fr], a.kl[o + q * 16 + fr]);
                        }
                    }
                }
            return;
        }
        // v heads: the cache rows, and the V^T planes from register pairs:
        // tokens m 16 + 4 fq + i (m even) and (m + 1) 16 + 4 fq + i fill
        // columns 8 fq .. 8 fq + 7 of the 32-key slice that starts at token
        // m 16 (the slice order of vt_column), one 16-byte store each.
#pragma unroll
        for (int m = 0; m < FM; ++m)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = t0 + wm + m * 16 + fq * 4 + i;
                if (t >= n) continue;
                KV *vc = reinterpret_cast<KV *>(a.v_cache) + (long long)head * a.head_stride +
                         (pos0 + t) * a.pos_stride;
#pragma unroll
                for (int q = 0; q < 8; ++q) store_kv(vc + q * 16 + fr, acc[m][q][i]);
            }
        if (a.vh) {
#pragma unroll
            for (int m = 0; m < FM; m += 2) {
                const int s0 = t0 + wm + m * 16;  // the slice's first token (pos0 + s0 is a multiple of 32)
                if (s0 >= n) continue;
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const long long o = ((long long)head * 128 + q * 16 + fr) * a.plane_len + pos0 + s0 + 8 * fq;
                    if (s0 + 32 <= n) {
                        uint2 h0, l0, h1, l1;
                        split_bf16x4(make_float4(acc[m][q][0], acc[m][q][1], acc[m][q][2], acc[m][q][3]), h0, l0);
                        split_bf16x4(
                            make_float4(acc[m + 1][q][0], acc[m + 1][q][1], acc[m + 1][q][2], acc[m + 1][q][3]), h1,
                            l1);
                        *reinterpret_cast<uint4 *>(a.vh + o) = make_uint4(h0.x, h0.y, h1.x, h1.y);
                        *reinterpret_cast<uint4 *>(a.vl + o) = make_uint4(l0.x, l0.y, l1.x, l1.y);
                    } else {
                        // The last slice, partly past the tokens: only their columns.
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const int tm = j < 4 ? m : m + 1;
                            if (t0 + wm + tm * 16 + fq * 4 + (j & 3) < n)
                                split_bf16(acc[tm][q][j & 3], a.vh[o + j], a.vl[o + j]);
                        }
                    }
                }
            }
        }
        return;
    }
    if constexpr (EPI == kQkvHead) {
        // The head's 128 columns of each token through LDS; then a wave per
        // token: q and k heads get RMSNorm + RoPE at their position (q back
        // to the attention's input, k to the cache), v heads go to the cache.
        constexpr int EPS = T::BN + 4;
        static_assert(T::BN == 128, "one head of 128 dimensions a tile");
        static_assert(sizeof(ring) >= sizeof(float) * T::BM * EPS, "the epilogue tile fits the ring");
        float *ep = reinterpret_cast<float *>(ring);
        __syncthreads();
#pragma unroll
        for (int m = 0; m < FM; ++m)
#pragma unroll
            for (int q = 0; q < FN; ++q)
#pragma unroll
                for (int i = 0; i < 4; ++i) ep[(wm + m * 16 + fq * 4 + i) * EPS + wn + q * 16 + fr] = acc[m][q][i];
        __syncthreads();
        const QkvPostArgs &a = *ht.a;
        const long long pos0 = a.pos_dev ? *a.pos_dev : a.pos;
        // A v head's V^T planes: a whole tile of 32 tokens that starts a
        // 32-key slice writes its slice from LDS, 16 bytes a store; other
        // tiles write each element at its column.
        const bool vt_tile = ht.role == 2 && a.vh && ((pos0 + t0) & 31) == 0 && t0 + T::BM <= n;
        if (vt_tile) {
            static_assert(T::BM == 32, "a tile of one 32-key slice");
            const long long c0 = pos0 + t0;
            for (int e = tid; e < 128 * 4; e += T::NT) {
                const int d = e >> 2, g = e & 3;
                float f[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) f[i] = ep[(i < 4 ? 4 * g + i : 16 + 4 * g + i - 4) * EPS + d];
                uint2 h0, l0, h1, l1;
                split_bf16x4(make_float4(f[0], f[1], f[2], f[3]), h0, l0);
                split_bf16x4(make_float4(f[4], f[5], f[6], f[7]), h1, l1);
                const long long o = ((long long)ht.head * 128 + d) * a.plane_len + c0 + 8 * g;
                *reinterpret_cast<uint4 *>(a.vh + o) = make_uint4(h0.x, h0.y, h1.x, h1.y);
                *reinterpret_cast<uint4 *>(a.vl + o) = make_uint4(l0.x, l0.y, l1.x, l1.y);
            }
        }
        for (int tl = wave; tl < T::BM; tl += T::NT / 64) {
            const long long t = t0 + tl;
            if (t >= n) break;
            float av[4] = {ep[tl * EPS + lane], 0.f, 0.f, 0.f}, bv[4] = {ep[tl * EPS + 64 + lane], 0.f, 0.f, 0.f};
            const long long pos = pos0 + t;
            if (ht.role == 2) {
                KV *vc = reinterpret_cast<KV *>(a.v_cache) + (long long)ht.head * a.head_stride + pos * a.pos_stride;
                store_kv(vc + lane, av[0]);
                store_kv(vc + lane + 64, bv[0]);
                if (a.vh && !vt_tile) {
                    // V^T planes: dimension-major rows, the key's column in its slice.
                    const long long col = (pos & ~31LL) + vt_column((int)(pos & 31));
                    const long long o0 = ((long long)ht.head * 128 + lane) * a.plane_len + col;
                    const long long o1 = o0 + 64 * a.plane_len;
                    split_bf16(av[0], a.vh[o0], a.vl[o0]);
                    split_bf16(bv[0], a.vh[o1], a.vl[o1]);
                }
                continue;
            }
            norm_rope_pairs(av, bv, lane, 128, ht.role == 0 ? a.q_norm : a.k_norm, a.eps, a.rope + pos * 128);
            if (ht.role == 0) {
                float *dst = a.q + (t * a.n_heads + ht.head) * 128;
                dst[lane] = av[0];
                dst[lane + 64] = bv[0];
            } else {
                KV *kc = reinterpret_cast<KV *>(a.k_cache) + (long long)ht.head * a.head_stride + pos * a.pos_stride;
                store_kv(kc + lane, av[0]);
                store_kv(kc + lane + 64, bv[0]);
                if (a.kh) {
                    // K planes: row-major, the key's row at its position.
                    const long long o = ((long long)ht.head * a.plane_len + pos) * 128 + lane;
                    split_bf16(av[0], a.kh[o], a.kl[o]);
                    split_bf16(bv[0], a.kh[o + 64], a.kl[o + 64]);
                }
            }
        }
        return;
    }
    const int rows = sg.rows;
    float *out = ksplit > 1 ? part + (size_t)z * n * rows : sg.out;
#pragma unroll
    for (int m = 0; m < FM; ++m)
#pragma unroll
        for (int q = 0; q < FN; ++q)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = t0 + wm + m * 16 + fq * 4 + i;
                if (t < n) out[(size_t)t * rows + rl + wn + q * 16 + fr] = acc[m][q][i];
            }
}

__global__ __launch_bounds__(Small::NT, 2) void gemm_kernel(int gxy, int rows0, const uint16_t *__restrict__ w0,
                                                        float *__restrict__ out0, const uint16_t *__restrict__ hi,
                                                        const uint16_t *__restrict__ lo, int n, int cols, int ksplit,
                                                        float *__restrict__ part, Segs sg) {
    int tx, ty;
    tile_of_block<8>(tx, ty, gxy & 0xffff, gxy >> 16);
    gemm_tile<Small>(ty, seg_tile(w0, out0, rows0, sg, tx * Small::BN), hi, lo, n, cols, part, ksplit);
}

__global__ __launch_bounds__(Large::NT, 1) void gemm_large_kernel(int gxy, int rows0, const uint16_t *__restrict__ w0,
                                                        float *__restrict__ out0, const uint16_t *__restrict__ hi,
                                                        const uint16_t *__restrict__ lo, int n, int cols, int ksplit,
                                                        float *__restrict__ part, Segs sg) {
    int tx, ty;
    tile_of_block<4>(tx, ty, gxy & 0xffff, gxy >> 16);
    gemm_tile<Large>(ty, seg_tile(w0, out0, rows0, sg, tx * Large::BN), hi, lo, n, cols, part, ksplit);
}

__global__ __launch_bounds__(Huge::NT, 1) void gemm_huge_kernel(int gxy, int rows0, const uint16_t *__restrict__ w0,
                                                        float *__restrict__ out0, const uint16_t *__restrict__ hi,
                                                        const uint16_t *__restrict__ lo, int n, int cols, int ksplit,
                                                        float *__restrict__ part, Segs sg) {
    int tx, ty;
    tile_of_block<2>(tx, ty, gxy & 0xffff, gxy >> 16);
    gemm_tile<Huge>(ty, seg_tile(w0, out0, rows0, sg, tx * Huge::BN), hi, lo, n, cols, part, ksplit);
}

// gate and up in one launch, block x taking rows [x BN/2, (x + 1) BN/2) of
// each, with the SiLU * up epilogue.
template <class T>
__global__ __launch_bounds__(T::NT, T::NT == 256 ? (T::kStages == 2 ? 3 : 2) : 1) void gemm_silu_kernel(
    const uint16_t *__restrict__ gate, const uint16_t *__restrict__ up, const uint16_t *__restrict__ hi,
    const uint16_t *__restrict__ lo, int n, int cols, int inter, int gx, int gy, uint16_t *__restrict__ h_hi,
    uint16_t *__restrict__ h_lo) {
    int tx, ty;
    tile_of_block<T::NT == 256 ? 8 : T::BM == 256 ? 2 : 4>(tx, ty, gx, gy);
    const PairTile pt{gate, up, h_hi, h_lo, inter, tx * (T::BN / 2)};
    gemm_tile<T, kSiluPairs>(ty, SegTile{}, hi, lo, n, cols, nullptr, 1, pt);
}

// q, k and v in one launch, block x taking attention head x of the
// concatenation (q heads, then k, then v) for 32 tokens, with the q/k/v
// post-processing epilogue (the work of qk_norm_rope_append).
template <typename KV>
__global__ __launch_bounds__(Head::NT, 2) void gemm_qkv_kernel(const uint16_t *__restrict__ wq,
                                                               const uint16_t *__restrict__ wk,
                                                               const uint16_t *__restrict__ wv,
                                                               const uint16_t *__restrict__ hi,
                                                               const uint16_t *__restrict__ lo, int n, int cols,
                                                               int gxy, int nqkv, QkvPostArgs a) {
    // gxy = grid x | grid y << 16, nqkv = q heads | KV heads << 16: packed so
    // that every field the first loads need fits the 14 preloaded dwords.
    const int nq = nqkv & 0xffff, nkv = nqkv >> 16;
    int h, ty;
    tile_of_block<8>(h, ty, gxy & 0xffff, gxy >> 16);
    const int role = h < nq ? 0 : h < nq + nkv ? 1 : 2;
    const int head = role == 0 ? h : role == 1 ? h - nq : h - nq - nkv;
    const uint16_t *w = (role == 0 ? wq : role == 1 ? wk : wv) + (size_t)head * 128 * cols;
    SegTile sg{w, nullptr, 128, 0};
    gemm_tile<Head, kQkvHead, KV>(ty, sg, hi, lo, n, cols, nullptr, 1, PairTile{}, HeadTile{&a, role, head});
}

// q, k and v in one launch on the 256 x 256 tile, block x taking rows
// [256 x, 256 x + 256) of the concatenation (two attention heads, one a
// wave of 64 tokens x 128 rows), with the q/k/v post-processing epilogue.
template <typename KV>
__global__ __launch_bounds__(Huge::NT, 1) void gemm_qkv_huge_kernel(const uint16_t *__restrict__ wq,
                                                                    const uint16_t *__restrict__ wk,
                                                                    const uint16_t *__restrict__ wv,
                                                                    const uint16_t *__restrict__ hi,
                                                                    const uint16_t *__restrict__ lo, int n, int cols,
                                                                    int gxy, int nqkv, QkvPostArgs a) {
    // Packed as in gemm_qkv_kernel.
    int tx, ty;
    tile_of_block<2>(tx, ty, gxy & 0xffff, gxy >> 16);
    const int qd = (nqkv & 0xffff) * 128, kvd = (nqkv >> 16) * 128, r0 = tx * Huge::BN;
    const int role = r0 < qd ? 0 : r0 < qd + kvd ? 1 : 2;
    const int local = role == 0 ? r0 : role == 1 ? r0 - qd : r0 - qd - kvd;
    const uint16_t *w = (role == 0 ? wq : role == 1 ? wk : wv) + (size_t)local * cols;
    SegTile sg{w, nullptr, Huge::BN, 0};
    gemm_tile<Huge, kQkvHeads, KV>(ty, sg, hi, lo, n, cols, nullptr, 1, PairTile{}, HeadTile{&a, role, local / 128});
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
    return rows % Small::BN == 0 && cols % BK == 0 && rows < ((size_t)1 << 24) && cols < ((size_t)1 << 20) &&
           rows * cols < ((size_t)1 << 40);
}

namespace {

// A launch takes the large tile when it has at least two large tiles a CU
// (and every matrix's rows are whole large tiles). Fewer leave the last round
// of one-block-a-CU tiles partly empty, and the small tile, two blocks a CU
// over four times the grid, finishes first (measured on the Qwen3 prefill
// shapes: 512 tokens x 19456 x 2560 203 against 180 us). With the XCD-aware
// tile order, two large tiles a CU already pay: a 2048-token Qwen3-0.6B
// prefill (its q/k/v GEMM, 512 large tiles) 9.26 -> 8.93 ms with the
// threshold at 512 rather than 768 tiles. A single matrix with one to three
// large tiles a CU and a deep K range (at least 96 steps) takes the large
// tile with K split in two (2048 tokens x 2560 x 9728: 311 against 346 us;
// with 64 steps, 2560 x 4096, the small tile stays ahead).
constexpr size_t kLargeMinTiles = 512;
constexpr size_t kLargeSplitMinTiles = 256;
// The 256 x 256 tile from three tiles a CU; a single matrix from one tile a
// CU, with K split in two (the Qwen3-4B o and down projections at 8192
// tokens, 320 tiles: 8192-token prefill 165.9 -> 160.6 ms against the
// 128 x 128 tile, K split in three 160.8, in four 161.9).
constexpr size_t kHugeMinTiles = 768;
// More small tiles than two a CU: the gate/up GEMM takes Small2.
constexpr size_t kSmall2MinTiles = 512;
constexpr size_t kHugeSplitMinTiles = 256;

struct Plan {
    bool large, huge;
    int ksplit;
};

// rows_large / rows_huge: every matrix's rows are whole large / huge tiles.
Plan gemm_plan(size_t n, size_t rows, size_t cols, int n_outs, bool rows_large, bool rows_huge) {
    const size_t nk = cols / BK;
    const size_t ht = rows_huge ? (rows / Huge::BN) * ((n + Huge::BM - 1) / Huge::BM) : 0;
    if (ht >= kHugeMinTiles) return {true, true, 1};
    if (n_outs == 1 && ht >= kHugeSplitMinTiles) return {true, true, 2};
    const size_t lt = rows_large ? (rows / Large::BN) * ((n + Large::BM - 1) / Large::BM) : 0;
    if (lt >= kLargeMinTiles) return {true, false, 1};
    if (n_outs == 1 && lt >= kLargeSplitMinTiles && nk >= 96) return {true, false, 2};
    if (n_outs != 1) return {false, false, 1};
    // Small tiles: a single matrix with few row tiles (o, down) splits K so
    // that the launch still fills the chip, keeping at least 4 K steps a split.
    const size_t tiles = (rows / Small::BN) * ((n + Small::BM - 1) / Small::BM);
    int ksplit = 1;
    while (ksplit < kGemmMaxSplitK && tiles * ksplit < 512 && (size_t)ksplit * 2 * 4 <= nk) ksplit *= 2;
    return {false, false, ksplit};
}

}  // namespace

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

int gemm_ksplit(size_t n, size_t rows, size_t cols, int n_outs) {
    // Only a single matrix splits K: its rows are the whole concatenation.
    return gemm_plan(n, rows, cols, n_outs, rows % Large::BN == 0, n_outs == 1 && rows % Huge::BN == 0).ksplit;
}

hipError_t launch_gemm_hl(hipStream_t s, const uint16_t *hi, const uint16_t *lo, size_t n, size_t cols,
                          const GemmOut *outs, int n_outs, float *part, int ksplit) {
    if (n == 0) return hipSuccess;
    if (n_outs < 1 || n_outs > 3 || !hi || !lo || (n + Small::BM - 1) / Small::BM > 65535 ||
        n > ((size_t)1 << 24) || ksplit < 1 || ksplit > kGemmMaxSplitK || (ksplit > 1 && (n_outs != 1 || !part)) ||
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
    if (total / Small::BN > 65535) return hipErrorInvalidValue;
    bool rows_large = true, rows_huge = true;
    for (int i = 0; i < n_outs; ++i) {
        rows_large = rows_large && outs[i].rows % Large::BN == 0;
        rows_huge = rows_huge && outs[i].rows % Huge::BN == 0;
    }
    const Plan plan = gemm_plan(n, total, cols, n_outs, rows_large, rows_huge);
    // The grid's x and y sizes travel packed in 16 bits each (both under
    // 65536 by the checks above).
    auto pack = [](const dim3 &g) { return (int)(g.x | g.y << 16); };
    if (plan.huge && plan.ksplit == ksplit) {
        dim3 grid((unsigned)(total / Huge::BN), (unsigned)((n + Huge::BM - 1) / Huge::BM), (unsigned)ksplit);
        const int gxy = pack(grid);
        gemm_huge_kernel<<<grid, Huge::NT, 0, s>>>(gxy, sg.rows[0], sg.w[0], sg.out[0], hi, lo, (int)n, (int)cols,
                                                        ksplit, part, sg);
    } else if (plan.large && !plan.huge && plan.ksplit == ksplit) {
        dim3 grid((unsigned)(total / Large::BN), (unsigned)((n + Large::BM - 1) / Large::BM), (unsigned)ksplit);
        const int gxy = pack(grid);
        gemm_large_kernel<<<grid, Large::NT, 0, s>>>(gxy, sg.rows[0], sg.w[0], sg.out[0], hi, lo, (int)n, (int)cols,
                                                         ksplit, part, sg);
    } else {
        dim3 grid((unsigned)(total / Small::BN), (unsigned)((n + Small::BM - 1) / Small::BM), (unsigned)ksplit);
        const int gxy = pack(grid);
        gemm_kernel<<<grid, Small::NT, 0, s>>>(gxy, sg.rows[0], sg.w[0], sg.out[0], hi, lo, (int)n, (int)cols,
                                                   ksplit, part, sg);
    }
    return hipGetLastError();
}

hipError_t launch_gemm_silu(hipStream_t s, const uint16_t *hi, const uint16_t *lo, size_t n, size_t cols,
                            const uint16_t *gate, const uint16_t *up, size_t inter, uint16_t *h_hi, uint16_t *h_lo) {
    if (n == 0) return hipSuccess;
    if (!hi || !lo || !gate || !up || !h_hi || !h_lo || !gemm_supported(inter, cols) || inter > ((size_t)1 << 24) ||
        n > ((size_t)1 << 24) || (n + Small::BM - 1) / Small::BM > 65535 || inter % (Large::BN / 2) ||
        ((uintptr_t)h_hi | (uintptr_t)h_lo) % 8)
        return hipErrorInvalidValue;
    const Plan plan = gemm_plan(n, 2 * inter, cols, 2, true, inter % (Huge::BN / 2) == 0);
    if (plan.huge) {
        dim3 grid((unsigned)(inter / (Huge::BN / 2)), (unsigned)((n + Huge::BM - 1) / Huge::BM));
        gemm_silu_kernel<Huge><<<grid, Huge::NT, 0, s>>>(gate, up, hi, lo, (int)n, (int)cols, (int)inter,
                                                          (int)grid.x, (int)grid.y, h_hi, h_lo);
    } else if (plan.large) {
        dim3 grid((unsigned)(inter / (Large::BN / 2)), (unsigned)((n + Large::BM - 1) / Large::BM));
        gemm_silu_kernel<Large><<<grid, Large::NT, 0, s>>>(gate, up, hi, lo, (int)n, (int)cols, (int)inter,
                                                           (int)grid.x, (int)grid.y, h_hi, h_lo);
    } else {
        dim3 grid((unsigned)(inter / (Small::BN / 2)), (unsigned)((n + Small::BM - 1) / Small::BM));
        if ((size_t)grid.x * grid.y > kSmall2MinTiles)
            gemm_silu_kernel<Small2><<<grid, Small2::NT, 0, s>>>(gate, up, hi, lo, (int)n, (int)cols, (int)inter,
                                                                 (int)grid.x, (int)grid.y, h_hi, h_lo);
        else
            gemm_silu_kernel<Small><<<grid, Small::NT, 0, s>>>(gate, up, hi, lo, (int)n, (int)cols, (int)inter,
                                                               (int)grid.x, (int)grid.y, h_hi, h_lo);
    }
    return hipGetLastError();
}

bool gemm_qkv_huge_fused(size_t n, size_t q_rows, size_t kv_rows, size_t cols, size_t head_dim, long long pos) {
    const size_t rows = q_rows + 2 * kv_rows;
    return head_dim == 128 && q_rows % Huge::BN == 0 && kv_rows % Huge::BN == 0 && gemm_supported(rows, cols) &&
           pos % 32 == 0 && gemm_plan(n, rows, cols, 3, rows % Large::BN == 0, true).huge;
}

hipError_t launch_gemm_qkv_huge(hipStream_t s, const uint16_t *hi, const uint16_t *lo, size_t cols,
                                const uint16_t *wq, const uint16_t *wk, const uint16_t *wv, const QkvPostArgs &a) {
    const size_t n = (size_t)a.n, qd = (size_t)a.n_heads * 128, kvd = (size_t)a.n_kv_heads * 128;
    if (a.n <= 0 || a.pos_dev || !hi || !lo || a.head_dim != 128 || !gemm_qkv_huge_fused(n, qd, kvd, cols, 128, a.pos) ||
        (a.kh && (!a.kl || !a.vh || !a.vl || a.plane_len % 64 || a.pos + a.n > a.plane_len)))
        return hipErrorInvalidValue;
    dim3 grid((unsigned)((qd + 2 * kvd) / Huge::BN), (unsigned)((n + Huge::BM - 1) / Huge::BM));
    if (grid.x > 0xffff || grid.y > 0xffff || a.n_heads > 0xffff || a.n_kv_heads > 0x7fff)
        return hipErrorInvalidValue;  // they travel packed in 16 bits
    const int gxy = (int)(grid.x | grid.y << 16), nqkv = a.n_heads | a.n_kv_heads << 16;
    if (a.kv_bf16)
        gemm_qkv_huge_kernel<uint16_t><<<grid, Huge::NT, 0, s>>>(wq, wk, wv, hi, lo, (int)n, (int)cols, gxy, nqkv, a);
    else
        gemm_qkv_huge_kernel<float><<<grid, Huge::NT, 0, s>>>(wq, wk, wv, hi, lo, (int)n, (int)cols, gxy, nqkv, a);
    return hipGetLastError();
}

bool gemm_qkv_fused(size_t n, size_t q_rows, size_t kv_rows, size_t cols, size_t head_dim) {
    return head_dim == 128 && q_rows % 128 == 0 && kv_rows % 128 == 0 && cols % BK == 0 &&
           !gemm_plan(n, q_rows + 2 * kv_rows, cols, 3, true, false).large;
}

hipError_t launch_gemm_qkv(hipStream_t s, const uint16_t *hi, const uint16_t *lo, size_t cols, const uint16_t *wq,
                           const uint16_t *wk, const uint16_t *wv, const QkvPostArgs &a) {
    if (a.n == 0) return hipSuccess;
    if (!hi || !lo || !wq || !wk || !wv || a.head_dim != 128 || cols % BK || cols >= ((size_t)1 << 20) ||
        a.n_heads < 1 || a.n_kv_heads < 1 || (a.n + Head::BM - 1) / Head::BM > 65535 ||
        a.n_heads + 2 * a.n_kv_heads > 0xffff)
        return hipErrorInvalidValue;
    // The planes as launch_gemm_qkv_huge takes them (a position read on the
    // device is the caller's to keep below plane_len).
    if (a.kh && (!a.kl || !a.vh || !a.vl || a.kv_bf16 || a.plane_len % 64 ||
                 (!a.pos_dev && (a.pos < 0 || a.pos + a.n > a.plane_len))))
        return hipErrorInvalidValue;
    dim3 grid((unsigned)(a.n_heads + 2 * a.n_kv_heads), (unsigned)((a.n + Head::BM - 1) / Head::BM));
    const int gxy = (int)(grid.x | grid.y << 16), nqkv = a.n_heads | a.n_kv_heads << 16;
    if (a.kv_bf16)
        gemm_qkv_kernel<uint16_t><<<grid, Head::NT, 0, s>>>(wq, wk, wv, hi, lo, a.n, (int)cols, gxy, nqkv, a);
    else
        gemm_qkv_kernel<float><<<grid, Head::NT, 0, s>>>(wq, wk, wv, hi, lo, a.n, (int)cols, gxy, nqkv, a);
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

hipError_t launch_gemm_outs(hipStream_t s, const float *x, size_t n, size_t cols, const GemmOut *outs, int n_outs) {
    if (n == 0) return hipSuccess;
    if (n_outs < 1 || n_outs > 3) return hipErrorInvalidValue;
    size_t most = 0;
    for (int i = 0; i < n_outs; ++i) {
        if (!gemm_supported(outs[i].rows, cols)) return hipErrorInvalidValue;
        most = std::max(most, outs[i].rows);
    }
    void *scratch = nullptr;
    const size_t bytes = gemm_scratch_bytes(n, cols, most);
    hipError_t e = hipMallocAsync(&scratch, bytes, s);
    if (e != hipSuccess) return e;
    e = launch_gemm_multi(s, x, n, cols, outs, n_outs, scratch, bytes);
    const hipError_t f = hipFreeAsync(scratch, s);
    return e != hipSuccess ? e : f;
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
