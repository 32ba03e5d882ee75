// Fused kernels of one greedy decode step (one token, batch 1), five per layer,
// captured once into a HIP graph and replayed at every position.
//
//   1 x = x_prev (+ y_prev) in every block, RMSNorm, q/k/v GEMV rows
//   2 per KV head: q/k RMSNorm, RoPE, KV append, attention over the cache
//   3 o GEMV rows (+ merge of attention splits)
//   4 x = x1 + o in every block, RMSNorm, gate and up rows, SiLU * up
//   5 down GEMV rows
// then the final RMSNorm with the output projection and a per-block argmax,
// and the pick. The residual stream is never updated in place: each kernel
// that adds to it reads one buffer and writes another, so every block can
// recompute the sum it needs.
//
// The GEMVs are HBM-bound: each block issues the 16-byte loads of all its
// weight rows first (they do not depend on the activations; non-temporal, as
// a step reads each weight once), then builds the normalized input in LDS
// while those loads are in flight, then reduces one row per wave with DPP.
#include <algorithm>

#include "common.h"
#include "device_util.h"
#include "step.h"
#include "step_dev.h"

namespace th {

namespace {

enum Prologue { kNormSum, kPlain };
enum Epilogue { kStore, kSiluPairs, kLogits };

struct GemvArgs {
    Rows rows;
    int n_rows;            // total rows
    int cols;
    const float *a, *b;    // input = a (+ b)
    const uint16_t *gain;  // RMSNorm gains (kNormSum)
    float eps;
    float *x_out;          // where the summed input is kept (kNormSum), or null
    float *out;            // kStore: out[r]; kSiluPairs: out[j] for rows (j, j + n_rows/2); kLogits: logits
    uint64_t *argmax;      // kLogits: per-block (key, inverted index) maxima
    // kStore with outs[0] set: the rows of matrix i of `rows` go to outs[i]
    // (q, k and v in buffers of their own) instead of out.
    float *outs[3];
};

// The fields a GEMV block needs for its first loads travel as leading scalar
// kernel arguments (the matrices' bases, the first two row counts, the rows
// and columns, the input vectors' addresses: 14 dwords, what gfx950
// preloads), which the code object asks to have preloaded into SGPRs at wave
// launch: the input and weight loads then issue without waiting on a fetch of
// the kernel arguments. The same fields stay in GemvArgs for the host side.
#define TH_GEMV_HEAD                                                                                       \
    const uint16_t *__restrict__ w0, const uint16_t *__restrict__ w1, const uint16_t *__restrict__ w2, int c0, \
        int c1, int n_rows, int cols, const float *__restrict__ in_a, const float *__restrict__ in_b

// The q/k/v GEMV and the q/k/v + attention launches lead with the three
// matrices' bases, the q and k row counts packed (q | k << 16; v has k's),
// the columns packed with the layer (cols | layer << 16), the input vectors'
// and the RMSNorm gains' addresses: 14 dwords, all preloaded, so that the
// GEMV blocks request their input, gains and weight rows without fetching a
// kernel argument.
#define TH_QKV_HEAD                                                                                        \
    const uint16_t *__restrict__ w0, const uint16_t *__restrict__ w1, const uint16_t *__restrict__ w2, int rows01, \
        int cols_layer, const float *__restrict__ in_a, const float *__restrict__ in_b,                         \
        const uint16_t *__restrict__ gain
#define TH_QKV_HEAD_OF(q, a) (a).rows.base[0], (a).rows.base[1], (a).rows.base[2], \
                             (a).rows.count[0] | (a).rows.count[1] << 16, (a).cols | (q).layer << 16, (a).a, (a).b, \
                             (a).gain
// Unpacks TH_QKV_HEAD's counts.
#define TH_QKV_HEAD_UNPACK                                                                          \
    const int c0 = rows01 & 0xffff, c1 = rows01 >> 16, n_rows = c0 + 2 * c1, cols = cols_layer & 0xffff, \
              layer = cols_layer >> 16

// Where kStore writes row r.
__device__ __forceinline__ float *store_at(const GemvArgs &a, int r) {
    if (!a.outs[0]) return a.out + r;
    if (r < a.rows.count[0]) return a.outs[0] + r;
    r -= a.rows.count[0];
    if (r < a.rows.count[1]) return a.outs[1] + r;
    return a.outs[2] + (r - a.rows.count[1]);
}

constexpr bool gemv_early_gain(Prologue pro, Epilogue epi) { return pro == kNormSum && epi != kStore; }

// One block: RPW rows per wave, CPL 16-byte chunks per lane per row. With
// EARLY, the RMSNorm gains (at `gain`) are requested with the input, ahead of
// the weight rows; otherwise after them, from a.gain.
// The matrices' table is built here from scalars: a table passed in by
// reference went to scratch memory, its row selection into a
// dynamically-indexed load.
template <int RPW, int CPL, Prologue PRO, Epilogue EPI, bool EARLY>
__device__ __forceinline__ void gemv_body(const uint16_t *w0, const uint16_t *w1, const uint16_t *w2, int c0, int c1,
                                          int n_rows, int cols, const float *in_a, const float *in_b,
                                          const uint16_t *gain, const GemvArgs &a) {
    static_assert(EPI != kSiluPairs || RPW % 2 == 0, "a wave holds whole (gate, up) pairs");
    constexpr bool kEarlyGain = EARLY;
    const Rows rows{{w0, w1, w2}, {c0, c1, 0}};
    extern __shared__ float xs[];
    __shared__ float red[kWaves];
    __shared__ uint64_t red64[kWaves];
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    constexpr int RPB = RPW * kWaves;
    const int r0 = blockIdx.x * RPB + wave * RPW;
    // For paired rows (gate j, up j), a wave takes j and j + half.
    const int half = n_rows / 2;
    // The input's requests go first (their addresses are preloaded): its
    // sum, and the RMSNorm's reduction, then wait only for them, while the
    // weight rows stream in behind.
    constexpr int NV = (CPL * 128 + kThreads - 1) / kThreads;
    InputRegs<NV> in;
    load_input(in, in_a, in_b, cols);
    if constexpr (kEarlyGain) load_gain(in, gain, cols);
    uint4 w[RPW][CPL];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        int row;
        if (EPI == kSiluPairs) row = (r & 1) ? (r0 + r - 1) / 2 + half : (r0 + r) / 2;
        else row = r0 + r;
        const bool valid = EPI == kSiluPairs ? (r0 + r - (r & 1)) / 2 < half : row < n_rows;
        const uint4 *p = row_at(rows, valid ? row : 0, cols);
#pragma unroll
        for (int c = 0; c < CPL; ++c) w[r][c] = ld_nt_row(p, c * 64 + lane);
    }
    if constexpr (PRO == kNormSum && !kEarlyGain) load_gain(in, a.gain, cols);
    finish_input<PRO == kNormSum>(in, xs, in_b != nullptr, cols, a.eps, a.x_out, red);
    float res[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) acc = dot8(xs, w[r][c], c * 64 + lane, acc);
        res[r] = wave_sum_dpp(acc);
    }
    if (EPI == kStore) {
        if (lane < RPW) {
#pragma unroll
            for (int r = 0; r < RPW; ++r)
                if (lane == r && r0 + r < n_rows) *store_at(a, r0 + r) = res[r];
        }
    } else if (EPI == kSiluPairs) {
        // Rows r0 + 2i and r0 + 2i + 1 of the wave are gate j and up j.
#pragma unroll
        for (int r = 0; r + 1 < RPW; r += 2) {
            const int j = (r0 + r) / 2;
            if (lane == 0 && j < half) a.out[j] = silu(res[r]) * res[r + 1];
        }
    } else {
        uint64_t best = 0;
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            if (r0 + r < n_rows) {
                if (lane == 0) a.out[r0 + r] = res[r];
                best = max_u64(best, argmax_pack(res[r], (uint32_t)(r0 + r)));
            }
        }
        if (lane == 0) red64[wave] = best;
        __syncthreads();
        if (tid == 0) {
            uint64_t b = 0;
            for (int i = 0; i < kWaves; ++i) b = max_u64(b, red64[i]);
            a.argmax[blockIdx.x] = b;
        }
    }
}

// The RMSNorm launches of one or two matrices (gate/up, the output
// projection) take the gains' address in the third matrix's slot and request
// them early.
template <int RPW, int CPL, Prologue PRO, Epilogue EPI>
__global__ __launch_bounds__(kThreads) void gemv_kernel(TH_GEMV_HEAD, GemvArgs a) {
    constexpr bool kEarlyGain = gemv_early_gain(PRO, EPI);
    // The gate/up launch of rows of at most two 512-column spans (one round
    // of blocks at the Qwen3-0.6B shape) with a CU's blocks at different
    // issue priorities, as the attention launches: Qwen3-0.6B step 0.5117 ->
    // 0.5094 ms over four paired runs (all faster). At five spans (Qwen3-4B,
    // two rounds of blocks) it was slower (2.1844 -> 2.2008 ms at 8192
    // positions), and so were the other GEMVs.
    if constexpr (EPI == kSiluPairs && CPL <= 2) {
        switch ((blockIdx.x >> 8) & 3) {
        case 0: __builtin_amdgcn_s_setprio(0); break;
        case 1: __builtin_amdgcn_s_setprio(1); break;
        case 2: __builtin_amdgcn_s_setprio(2); break;
        default: __builtin_amdgcn_s_setprio(3); break;
        }
    }
    gemv_body<RPW, CPL, PRO, EPI, kEarlyGain>(w0, w1, kEarlyGain ? nullptr : w2, c0, c1, n_rows, cols, in_a, in_b, w2,
                                              a);
}

// The q/k/v GEMV (RMSNorm, three matrices) with the head of the q/k/v +
// attention launches, whose gains' address it requests early.
template <int RPW, int CPL>
__global__ __launch_bounds__(kThreads) void gemv_qkv_kernel(TH_QKV_HEAD, GemvArgs a) {
    TH_QKV_HEAD_UNPACK;
    (void)layer;
    gemv_body<RPW, CPL, kNormSum, kStore, true>(w0, w1, w2, c0, c1, n_rows, cols, in_a, in_b, gain, a);
}

// Whether TH_QKV_HEAD's packed fields hold a q/k/v GEMV's counts (k and v
// rows equal; rows and columns below 2^16).
bool qkv_rows_pack(const GemvArgs &a) {
    return a.rows.count[0] > 0 && a.rows.count[0] < 65536 && a.rows.count[1] > 0 && a.rows.count[1] < 32768 &&
           a.rows.count[2] == a.rows.count[1] && a.n_rows == a.rows.count[0] + 2 * a.rows.count[1] &&
           a.cols < 65536;
}

template <int RPW, int CPL, Prologue PRO, Epilogue EPI>
hipError_t gemv_launch(hipStream_t s, const GemvArgs &a) {
    constexpr int RPB = RPW * kWaves;
    dim3 grid((unsigned)((a.n_rows + RPB - 1) / RPB));
    const size_t lds = a.cols * sizeof(float);
    if constexpr (PRO == kNormSum && EPI == kStore) {
        if (!qkv_rows_pack(a)) return hipErrorInvalidValue;
        gemv_qkv_kernel<RPW, CPL><<<grid, kThreads, lds, s>>>(
            a.rows.base[0], a.rows.base[1], a.rows.base[2], a.rows.count[0] | a.rows.count[1] << 16, a.cols, a.a, a.b,
            a.gain, a);
    } else {
        if (gemv_early_gain(PRO, EPI) && a.rows.count[0] + a.rows.count[1] != a.n_rows) return hipErrorInvalidValue;
        gemv_kernel<RPW, CPL, PRO, EPI><<<grid, kThreads, lds, s>>>(
            a.rows.base[0], a.rows.base[1], gemv_early_gain(PRO, EPI) ? a.gain : a.rows.base[2], a.rows.count[0],
            a.rows.count[1], a.n_rows, a.cols, a.a, a.b, a);
    }
    return hipGetLastError();
}

// Dispatch on chunks per lane (cols / 512). Rows of 19 chunks (the 9728
// columns of the Qwen3-4B down projection) keep one row a wave, or two for the
// paired SiLU epilogue, to bound the registers that hold them; the output
// projection's argmax partials assume four rows a wave, so its columns never
// take that case (step_supported keeps hidden sizes to at most 8 chunks).
template <int RPW, Prologue PRO, Epilogue EPI>
hipError_t gemv_dispatch(hipStream_t s, const GemvArgs &a) {
    static_assert(EPI != kLogits || RPW == 4, "the argmax partials count blocks of four rows a wave");
    switch (a.cols / 512) {
    case 1: return gemv_launch<RPW, 1, PRO, EPI>(s, a);
    case 2: return gemv_launch<RPW, 2, PRO, EPI>(s, a);
    case 3: return gemv_launch<RPW, 3, PRO, EPI>(s, a);
    case 4: return gemv_launch<RPW, 4, PRO, EPI>(s, a);
    case 5: return gemv_launch<RPW, 5, PRO, EPI>(s, a);
    case 6: return gemv_launch<RPW, 6, PRO, EPI>(s, a);
    case 8: return gemv_launch<RPW, 8, PRO, EPI>(s, a);
    case 19:
        if (EPI == kLogits) return hipErrorInvalidValue;
        return gemv_launch<(RPW == 1 ? 1 : EPI == kSiluPairs ? 2 : 1), 19, PRO, EPI>(s, a);
    default: return hipErrorInvalidValue;
    }
}

// The q/k/v rows of launch_step_qkv published as epoch words by the first
// blocks, and after them one block per q head and chunk of the cache that
// attends from those words. Blocks start in index order and the GEMV blocks
// never wait, so the attention blocks' polls always end.
// Rows a wave of the q/k/v GEMV blocks (Qwen3-0.6B step: 0.6114 ms with 2,
// 0.6094 with 4, 0.645 with 1; with the branch-free P.V loop, 0.5990 with 4
// and 0.5975 with 5; with non-temporal weight loads, 0.5673 / 0.5651 /
// 0.5640 / 0.5693 ms with 2 / 3 / 4 / 5; with the input requested ahead of
// the weights, 0.5145 / 0.5178 / 0.5113 ms with 3 / 4 / 5, while five slowed
// the streaming launch at 4K positions, 0.761 -> 0.804 ms, and the Qwen3-4B
// shape, 1.674 -> 1.717 ms).
constexpr int kQkvRowsPerWave = 4;
// Those of qkv_attn_kernel for rows of CPL 512-column spans.
template <int CPL>
constexpr int qkv_attn_rows_per_wave() {
    return CPL <= 2 ? 5 : kQkvRowsPerWave;
}

// The GEMV blocks of the q/k/v + attention launches: the q/k/v rows of
// launch_step_qkv, published as (value | epoch << 32) words.
template <int CPL, int RPW>
__device__ __forceinline__ void qkv_publish(const StepQkvAttnArgs &q, const GemvArgs &a, const Rows &rows, int n_rows,
                                            int cols, const float *in_a, const float *in_b, const uint16_t *gain,
                                            int layer) {
    constexpr int RPB = RPW * kWaves;
    extern __shared__ float xs[];
    __shared__ float red[kWaves];
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int r0 = blockIdx.x * RPB + wave * RPW;
    // The input and its gains first, then the weight rows (as gemv_kernel).
    constexpr int NV = (CPL * 128 + kThreads - 1) / kThreads;
    InputRegs<NV> in;
    load_input(in, in_a, in_b, cols);
    load_gain(in, gain, cols);
    uint4 w[RPW][CPL];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const uint4 *p = row_at(rows, r0 + r < n_rows ? r0 + r : 0, cols);
#pragma unroll
        for (int c = 0; c < CPL; ++c) w[r][c] = ld_nt_row(p, c * 64 + lane);
    }
    finish_input<true>(in, xs, in_b != nullptr, cols, a.eps, a.x_out, red);
    float res[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) acc = dot8(xs, w[r][c], c * 64 + lane, acc);
        res[r] = wave_sum_dpp(acc);
    }
    // The epoch, read only now: the weight requests above wait on nothing.
    const unsigned epoch = q.st->epoch * 64u + (unsigned)layer + 1u;
#pragma unroll
    for (int r = 0; r < RPW; ++r)
        if (lane == r && r0 + r < n_rows)
            __hip_atomic_store(q.words + r0 + r, ((unsigned long long)epoch << 32) | __float_as_uint(res[r]),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int CPL, int G, typename KV>
__global__ __launch_bounds__(kThreads) void qkv_attn_kernel(TH_QKV_HEAD, StepQkvAttnArgs q, GemvArgs a) {
    // The blocks a CU holds at once (256 apart: 8 XCDs x 32 CUs, dealt in
    // turn) at different issue priorities, as in the streaming attention:
    // Qwen3-0.6B step 0.5120 -> 0.5094 ms over four paired runs (all
    // faster). The same in the GEMVs and in the q/k/v + streaming launch was
    // slower.
    switch ((blockIdx.x >> 8) & 3) {
    case 0: __builtin_amdgcn_s_setprio(0); break;
    case 1: __builtin_amdgcn_s_setprio(1); break;
    case 2: __builtin_amdgcn_s_setprio(2); break;
    default: __builtin_amdgcn_s_setprio(3); break;
    }
    constexpr int RPW = qkv_attn_rows_per_wave<CPL>(), RPB = RPW * kWaves;
    TH_QKV_HEAD_UNPACK;
    const int ngemv = (n_rows + RPB - 1) / RPB;
    if ((int)blockIdx.x >= ngemv) {
        const unsigned epoch = q.st->epoch * 64u + (unsigned)layer + 1u;
        // `chunks` blocks per q head, one per pass of cached rows: the heads
        // of a KV group attend in parallel (each reads the group's rows), the
        // group's first head appends; each head's first chunk merges. The
        // heads are dealt so that a group's heads are (n_heads / G) * chunks
        // blocks apart: with 8 KV groups a multiple of 8, so that blocks,
        // which go to the 8 XCDs in turn by index, put a group's chunk c on
        // one XCD and its heads share that XCD's L2 for the group's rows and
        // k/v words (Qwen3-0.6B step, one chunk: 0.5128 -> 0.4979 ms; with
        // heads in order only 16 chunks placed them so, by chance).
        const int b = blockIdx.x - ngemv, hp = b / q.chunks, c = b % q.chunks;
        const int groups = q.at.n_heads / G, h = (hp % groups) * G + hp / groups, g = h / G;
        unsigned long long *xw = q.words + q.qkv.q_rows + 2 * q.qkv.kv_rows;
        attend_wave4<KV>(q.at, g, h, h % G == 0, c, q.words, epoch, q.err, xw, q.chunks);
        return;
    }
    qkv_publish<CPL, RPW>(q, a, Rows{{w0, w1, w2}, {c0, c1, 0}}, n_rows, cols, in_a, in_b, gain, layer);
}

template <int CPL, int G>
hipError_t qkv_attn_launch(hipStream_t s, const StepQkvAttnArgs &q, const GemvArgs &a) {
    constexpr int RPB = qkv_attn_rows_per_wave<CPL>() * kWaves;
    dim3 grid((unsigned)((a.n_rows + RPB - 1) / RPB + q.at.n_heads * q.chunks));
    const size_t lds = (size_t)a.cols * sizeof(float);
    if (q.at.kv_bf16)
        qkv_attn_kernel<CPL, G, uint16_t><<<grid, kThreads, lds, s>>>(TH_QKV_HEAD_OF(q, a), q, a);
    else
        qkv_attn_kernel<CPL, G, float><<<grid, kThreads, lds, s>>>(TH_QKV_HEAD_OF(q, a), q, a);
    return hipGetLastError();
}

template <int CPL>
hipError_t qkv_attn_g(hipStream_t s, const StepQkvAttnArgs &q, const GemvArgs &a) {
    switch (q.at.n_heads / q.at.n_kv_heads) {
    case 2: return qkv_attn_launch<CPL, 2>(s, q, a);
    case 4: return qkv_attn_launch<CPL, 4>(s, q, a);
    default: return hipErrorInvalidValue;
    }
}

// Waves a SIMD the streaming attention is built for: the most that keeps its
// two register sets of rows and its 16 G accumulators without spills (f32
// rows: 115 / 124 / 162 / 251 VGPRs for groups of 1 / 2 / 4 / 8 q heads).
template <int G, typename KV>
constexpr int stream_waves_per_eu() {
    return G <= 2 ? 4 : G == 4 ? 3 : 2;
}

// One block per (KV head, split of `chunk` positions), the rows streamed
// through registers in double-buffered passes. The fields its first requests
// need lead as preloaded arguments (13 dwords): the caches' bases, the raw
// q/k/v rows, the q/k gains, the head stride, nsplit | chunk << 9 and
// n_heads | n_kv_heads << 16 (Qwen3-4B at 8192 positions, with those requests
// ahead of the position's read: 2.2418 -> 2.2247 ms a step).
template <int G, typename KV>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(stream_waves_per_eu<G, KV>())))
void step_attention_stream_kernel(const void *__restrict__ k_cache, const void *__restrict__ v_cache,
                                  const float *__restrict__ qkv, const uint16_t *__restrict__ q_norm,
                                  const uint16_t *__restrict__ k_norm, int head_stride, int split_chunk, int heads,
                                  StepAttnArgs a) {
    // The blocks a CU holds at once at different issue priorities, so that
    // the waves a SIMD holds do not all reach their arithmetic together: the
    // favoured one computes while the others wait for rows. Blocks go to the
    // 8 XCDs in turn and to an XCD's 32 CUs in turn, so a CU's blocks are
    // 256 apart and the priority follows blockIdx.x / 256. Qwen3-4B at 8192
    // positions, six paired runs each: 2.1900 -> 2.1835 ms a step with the
    // priority following blockIdx.x % 4 (a CU's blocks then share one), and
    // 2.1817 -> 2.1787 ms from that to blockIdx.x / 256.
    switch ((blockIdx.x >> 8) & 3) {
    case 0: __builtin_amdgcn_s_setprio(0); break;
    case 1: __builtin_amdgcn_s_setprio(1); break;
    case 2: __builtin_amdgcn_s_setprio(2); break;
    default: __builtin_amdgcn_s_setprio(3); break;
    }
    const StreamHead e{k_cache, v_cache, qkv, q_norm, k_norm, head_stride, heads & 0xffff, heads >> 16};
    const int nsplit = split_chunk & 0x1ff;
    attend_stream<G, KV, false>(a, blockIdx.x / nsplit, blockIdx.x % nsplit, split_chunk >> 9, nullptr, 0, nullptr,
                                &e);
}

// The GEMV blocks of qkv_attn_kernel, then one streaming attention block per
// (KV head, split), which requests its first pass's rows and then polls the
// words: the launch for contexts past the chunked launch's reach, leaving
// the split partials for launch_attn_combine. Blocks start in index order
// and the GEMV blocks never wait, so the attention blocks' polls always end.
template <int CPL, int G, typename KV>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(stream_waves_per_eu<G, KV>())))
void qkv_stream_kernel(TH_QKV_HEAD, StepQkvAttnArgs q, GemvArgs a, long long chunk) {
    constexpr int RPB = kQkvRowsPerWave * kWaves;
    TH_QKV_HEAD_UNPACK;
    const int ngemv = (n_rows + RPB - 1) / RPB;
    if ((int)blockIdx.x >= ngemv) {
        const unsigned epoch = q.st->epoch * 64u + (unsigned)layer + 1u;
        const int b = blockIdx.x - ngemv;
        attend_stream<G, KV, true>(q.at, b / q.at.nsplit, b % q.at.nsplit, chunk, q.words, epoch, q.err);
        return;
    }
    qkv_publish<CPL, kQkvRowsPerWave>(q, a, Rows{{w0, w1, w2}, {c0, c1, 0}}, n_rows, cols, in_a, in_b, gain, layer);
}

template <int CPL, int G>
hipError_t qkv_stream_launch(hipStream_t s, const StepQkvAttnArgs &q, const GemvArgs &a) {
    constexpr int RPB = kQkvRowsPerWave * kWaves;
    const long long chunk = step_attention_chunk((size_t)(q.at.head_stride / 128), q.at.kv_bf16, q.at.nsplit);
    dim3 grid((unsigned)((a.n_rows + RPB - 1) / RPB + q.at.n_kv_heads * q.at.nsplit));
    const size_t lds = (size_t)a.cols * sizeof(float);
    if (q.at.kv_bf16)
        qkv_stream_kernel<CPL, G, uint16_t><<<grid, kThreads, lds, s>>>(TH_QKV_HEAD_OF(q, a), q, a, chunk);
    else
        qkv_stream_kernel<CPL, G, float><<<grid, kThreads, lds, s>>>(TH_QKV_HEAD_OF(q, a), q, a, chunk);
    return hipGetLastError();
}

template <int G>
hipError_t attn_stream_launch(hipStream_t s, const StepAttnArgs &a) {
    const long long max_len = a.head_stride / 128;
    const long long chunk = step_attention_chunk((size_t)max_len, a.kv_bf16, a.nsplit);
    // The packed arguments' ranges: at most 256 splits of fewer than 2^22
    // positions, a head stride and head counts that fit their words.
    if (a.nsplit < 1 || a.nsplit > 256 || chunk <= 0 || chunk >= (1LL << 22) || a.head_stride <= 0 ||
        a.head_stride > 0x7fffffffLL || a.n_heads <= 0 || a.n_heads >= 65536 || a.n_kv_heads <= 0 ||
        a.n_kv_heads >= 32768)
        return hipErrorInvalidValue;
    dim3 grid((unsigned)(a.n_kv_heads * a.nsplit));
    const int split_chunk = a.nsplit | (int)chunk << 9, heads = a.n_heads | a.n_kv_heads << 16;
    if (a.kv_bf16)
        step_attention_stream_kernel<G, uint16_t><<<grid, kThreads, 0, s>>>(
            a.k_cache, a.v_cache, a.qkv, a.q_norm, a.k_norm, (int)a.head_stride, split_chunk, heads, a);
    else
        step_attention_stream_kernel<G, float><<<grid, kThreads, 0, s>>>(
            a.k_cache, a.v_cache, a.qkv, a.q_norm, a.k_norm, (int)a.head_stride, split_chunk, heads, a);
    return hipGetLastError();
}

}  // namespace

bool step_supported(int hidden, int intermediate, int n_heads, int n_kv_heads, int head_dim) {
    if (head_dim != 128 || n_kv_heads <= 0 || n_heads % n_kv_heads) return false;
    const int g = n_heads / n_kv_heads;
    if (g != 1 && g != 2 && g != 4 && g != 8) return false;
    // Input lengths of the GEMVs: hidden (q/k/v, gate/up, output projection),
    // n_heads * head_dim (o) and intermediate (down); only the down projection
    // takes rows of 19 chunks (9728 columns).
    const int cols[3] = {hidden, n_heads * head_dim, intermediate};
    for (int i = 0; i < 3; ++i) {
        if (cols[i] % 512) return false;
        const int cpl = cols[i] / 512;
        if (cpl > 8 && !(i == 2 && cpl == 19)) return false;
    }
    return true;
}

hipError_t launch_step_qkv(hipStream_t s, const StepQkvArgs &q) {
    GemvArgs a{};
    a.rows.base[0] = q.wq;
    a.rows.count[0] = q.q_rows;
    a.rows.base[1] = q.wk;
    a.rows.count[1] = q.kv_rows;
    a.rows.base[2] = q.wv;
    a.rows.count[2] = q.kv_rows;
    a.n_rows = q.q_rows + 2 * q.kv_rows;
    a.cols = q.hidden;
    a.a = q.x_prev;
    a.b = q.y_prev;
    a.gain = q.gain;
    a.eps = q.eps;
    a.x_out = q.x_out;
    a.out = q.qkv;
    // Three rows a wave: Qwen3-4B at 8192 positions (the streaming step's
    // q/k/v launch, 512 blocks) 2.2023 -> 2.1988 ms a step over four paired
    // runs, against 2.2278 with one and 2.2186 with four.
    return gemv_dispatch<3, kNormSum, kStore>(s, a);
}

hipError_t launch_step_gemv(hipStream_t s, const uint16_t *w, int rows, int cols, const float *x, float *out) {
    GemvArgs a{};
    a.rows.base[0] = w;
    a.rows.count[0] = rows;
    a.n_rows = rows;
    a.cols = cols;
    a.a = x;
    a.out = out;
    return gemv_dispatch<1, kPlain, kStore>(s, a);
}

bool step_gemv_supported(int cols) {
    const int cpl = cols / 512;
    return cols > 0 && cols % 512 == 0 && (cpl <= 6 || cpl == 8 || cpl == 19);
}

hipError_t launch_step_gemv3(hipStream_t s, const uint16_t *const w[3], const int rows[3], int cols, const float *x,
                             float *const out[3]) {
    GemvArgs a{};
    for (int i = 0; i < 3; ++i) {
        a.rows.base[i] = w[i];
        a.rows.count[i] = rows[i];
        a.outs[i] = out[i];
        a.n_rows += rows[i];
    }
    a.cols = cols;
    a.a = x;
    return gemv_dispatch<2, kPlain, kStore>(s, a);
}

hipError_t launch_step_silu(hipStream_t s, const uint16_t *gate, const uint16_t *up, int inter, int cols,
                            const float *x, float *h) {
    GemvArgs a{};
    a.rows.base[0] = gate;
    a.rows.count[0] = inter;
    a.rows.base[1] = up;
    a.rows.count[1] = inter;
    a.n_rows = 2 * inter;
    a.cols = cols;
    a.a = x;
    a.out = h;
    return gemv_dispatch<2, kPlain, kSiluPairs>(s, a);
}

hipError_t launch_step_gate_up(hipStream_t s, const uint16_t *gate, const uint16_t *up, int inter, int hidden,
                               const float *x1, const float *o, const uint16_t *gain, float eps, float *x_out,
                               float *h) {
    GemvArgs a{};
    a.rows.base[0] = gate;
    a.rows.count[0] = inter;
    a.rows.base[1] = up;
    a.rows.count[1] = inter;
    a.n_rows = 2 * inter;
    a.cols = hidden;
    a.a = x1;
    a.b = o;
    a.gain = gain;
    a.eps = eps;
    a.x_out = x_out;
    a.out = h;
    // Four rows a wave where that still leaves 1024 blocks or more: each block
    // builds the normalized input once for twice the rows (Qwen3-4B, 1216
    // blocks: 1.808 -> 1.795 ms a step at a 16-token context, 2.371 -> 2.364
    // ms at 8192 positions); below that, two (Qwen3-0.6B: 768 blocks of two
    // against 384 of four, 0.552 against 0.565 ms).
    if (2 * inter / (4 * kWaves) >= 1024) return gemv_dispatch<4, kNormSum, kSiluPairs>(s, a);
    return gemv_dispatch<2, kNormSum, kSiluPairs>(s, a);
}

hipError_t launch_step_logits(hipStream_t s, const uint16_t *w, int vocab, int hidden, const float *x,
                              const float *y, const uint16_t *gain, float eps, float *logits, uint64_t *partials,
                              int *n_partials) {
    GemvArgs a{};
    a.rows.base[0] = w;
    a.rows.count[0] = vocab;
    a.n_rows = vocab;
    a.cols = hidden;
    a.a = x;
    a.b = y;
    a.gain = gain;
    a.eps = eps;
    a.out = logits;
    a.argmax = partials;
    *n_partials = (vocab + 4 * kWaves - 1) / (4 * kWaves);
    return gemv_dispatch<4, kNormSum, kLogits>(s, a);
}

int step_logits_partials(int vocab) { return (vocab + 4 * kWaves - 1) / (4 * kWaves); }

bool step_qkv_attn_supported(int hidden, int n_heads, int n_kv_heads) {
    if (n_kv_heads <= 0 || n_heads % n_kv_heads) return false;
    const int g = n_heads / n_kv_heads, cpl = hidden / 512;
    return hidden % 512 == 0 && (g == 2 || g == 4) && (cpl == 1 || cpl == 2 || cpl == 5);
}

int step_qkv_attn_chunks(size_t max_len, int kv_bf16, int n_heads) {
    const size_t rows = kv_bf16 ? KvRegs<uint16_t>::kRows : KvRegs<float>::kRows;
    const size_t chunks = (max_len + rows - 1) / rows;
    return chunks >= 1 && chunks <= (size_t)kStepQkvAttnMaxChunks &&
                   chunks * (size_t)n_heads <= (size_t)kStepQkvAttnMaxBlocks
               ? (int)chunks
               : 0;
}

int step_qkv_attn_rows(int kv_bf16) { return kv_bf16 ? KvRegs<uint16_t>::kRows : KvRegs<float>::kRows; }

size_t step_qkv_attn_words(int q_rows, int kv_rows, int n_heads, int chunks) {
    return (size_t)q_rows + 2 * (size_t)kv_rows + (size_t)n_heads * chunks * (128 + 2);
}

namespace {

GemvArgs qkv_gemv_args(const StepQkvArgs &k) {
    GemvArgs a{};
    a.rows.base[0] = k.wq;
    a.rows.count[0] = k.q_rows;
    a.rows.base[1] = k.wk;
    a.rows.count[1] = k.kv_rows;
    a.rows.base[2] = k.wv;
    a.rows.count[2] = k.kv_rows;
    a.n_rows = k.q_rows + 2 * k.kv_rows;
    a.cols = k.hidden;
    a.a = k.x_prev;
    a.b = k.y_prev;
    a.gain = k.gain;
    a.eps = k.eps;
    a.x_out = k.x_out;
    return a;
}

// Whether TH_QKV_HEAD's packed fields hold the launch's counts: rows and
// columns below 2^16; layer + 1 < 64, which also keeps the epoch words of
// successive steps apart.
bool qkv_head_packs(const StepQkvAttnArgs &q) {
    return q.qkv.q_rows > 0 && q.qkv.q_rows < 65536 && q.qkv.kv_rows > 0 && q.qkv.kv_rows < 32768 &&
           q.qkv.hidden < 65536 && q.layer >= 0 && q.layer < 63;
}

}  // namespace

hipError_t launch_step_qkv_stream(hipStream_t s, const StepQkvAttnArgs &q) {
    const StepQkvArgs &k = q.qkv;
    if (!step_qkv_attn_supported(k.hidden, q.at.n_heads, q.at.n_kv_heads) || !qkv_head_packs(q) ||
        q.at.nsplit < 1 || (q.at.nsplit > 1 && (!q.at.part_acc || !q.at.part_ml)) || (q.at.nsplit == 1 && !q.at.out))
        return hipErrorInvalidValue;
    const GemvArgs a = qkv_gemv_args(k);
    const int g = q.at.n_heads / q.at.n_kv_heads;
    switch (k.hidden / 512) {
    case 1: return g == 2 ? qkv_stream_launch<1, 2>(s, q, a) : qkv_stream_launch<1, 4>(s, q, a);
    case 2: return g == 2 ? qkv_stream_launch<2, 2>(s, q, a) : qkv_stream_launch<2, 4>(s, q, a);
    case 5: return g == 2 ? qkv_stream_launch<5, 2>(s, q, a) : qkv_stream_launch<5, 4>(s, q, a);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_step_qkv_attn(hipStream_t s, const StepQkvAttnArgs &q) {
    const StepQkvArgs &k = q.qkv;
    const long long max_len = q.at.head_stride / 128;
    if (!step_qkv_attn_supported(k.hidden, q.at.n_heads, q.at.n_kv_heads) || !qkv_head_packs(q) ||
        q.at.nsplit != 1 || q.chunks < 1 || q.chunks > kStepQkvAttnMaxChunks ||
        q.chunks * q.at.n_heads > kStepQkvAttnMaxBlocks ||
        (long long)(q.chunks - 1) * (q.at.kv_bf16 ? KvRegs<uint16_t>::kRows : KvRegs<float>::kRows) >= max_len)
        return hipErrorInvalidValue;
    const GemvArgs a = qkv_gemv_args(k);
    switch (k.hidden / 512) {
    case 1: return qkv_attn_g<1>(s, q, a);
    case 2: return qkv_attn_g<2>(s, q, a);
    case 5: return qkv_attn_g<5>(s, q, a);
    default: return hipErrorInvalidValue;
    }
}

// Rows of one pass of the streaming attention's block (four waves of 8 rows).
constexpr long long kStreamPassF32 = 32, kStreamPassBf16 = 32;

long long step_attention_chunk(size_t max_len, int kv_bf16, int nsplit) {
    const long long pass = kv_bf16 ? kStreamPassBf16 : kStreamPassF32;
    const long long c = ((long long)max_len + nsplit - 1) / nsplit;
    return (c + pass - 1) / pass * pass;
}

int step_stream_slots(int group, int kv_bf16, int num_cus) {
    int per_cu;
    switch (group) {
    case 1: per_cu = kv_bf16 ? stream_waves_per_eu<1, uint16_t>() : stream_waves_per_eu<1, float>(); break;
    case 2: per_cu = kv_bf16 ? stream_waves_per_eu<2, uint16_t>() : stream_waves_per_eu<2, float>(); break;
    case 4: per_cu = kv_bf16 ? stream_waves_per_eu<4, uint16_t>() : stream_waves_per_eu<4, float>(); break;
    default: per_cu = kv_bf16 ? stream_waves_per_eu<8, uint16_t>() : stream_waves_per_eu<8, float>(); break;
    }
    return std::max(num_cus, 1) * per_cu;
}

int step_attention_splits(size_t max_len, int kv_bf16, int group, int n_kv_heads, int num_cus) {
    if (max_len <= 512 || n_kv_heads < 1) return 1;
    // As many splits as fill the chip's block slots in one round (blocks a
    // CU = waves a SIMD the kernel is built for), in whole passes: a second,
    // partial round of blocks would leave most of the chip idle at its end
    // (Qwen3-4B at 8192 positions, f32: splits of 1 / 2 / 3 / 4 / 8 passes
    // gave 2.618 / 2.532 / 2.501 / 2.616 / 2.716 ms a step; three, 704
    // blocks for 768 slots, filled it).
    const long long want = std::max(1LL, (long long)step_stream_slots(group, kv_bf16, num_cus) / n_kv_heads);
    long long chunk = step_attention_chunk(max_len, kv_bf16, (int)std::min(want, 256LL));
    return (int)(((long long)max_len + chunk - 1) / chunk);
}

hipError_t launch_step_attention(hipStream_t s, const StepAttnArgs &a) {
    switch (a.n_heads / a.n_kv_heads) {
    case 1: return attn_stream_launch<1>(s, a);
    case 2: return attn_stream_launch<2>(s, a);
    case 4: return attn_stream_launch<4>(s, a);
    case 8: return attn_stream_launch<8>(s, a);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace th
