// The XCD-parallel decode kernel: every step of a greedy decode (model/chat.rs:
// 149-178 at temperature 0, each step one pass of model/model.rs:93-149 for one
// token) in one cooperative launch of one block per CU.
//
// Layout. An MI355X has eight XCDs of 32 CUs, each with its own L2. Block b
// runs on XCD b % 8 (checked at start). Each layer is split over the XCDs the
// way tensor parallelism splits it over devices: XCD g owns KV head g, the q
// heads of its group, its slice of the MLP (rows g I/8 .. of gate/up, the same
// columns of down) and the matching columns of o. Inside an XCD its 32 blocks
// share rows. The residual stream is replicated: every block holds all of x.
//
// Exchanges carry (f32 bits | epoch << 32) words, so data and readiness travel
// together and no fence is needed. Words read only inside the XCD that wrote
// them go through its L2 (workgroup-scope stores, loads that skip the CU's L1),
// about 3x faster than a device-wide exchange; the two all-reduces of a layer
// (after o and after down) cross XCDs with agent-scope words. Per layer:
//
//   A  RMSNorm(x) and this block's q/k/v rows of the group   -> qkv  (in XCD)
//   B  blocks 0..nsplit-1: q/k RMSNorm + RoPE, attention over
//      their split of the positions, KV append               -> partials (in XCD)
//   C  merge the partials, this block's rows of o restricted
//      to the group's columns                                -> o partial (all XCDs)
//      all-reduce: sum the eight partials of this block's
//      residual rows, add, share inside the XCD               -> x
//   D  RMSNorm(x), gate/up pairs of the XCD's slice, SiLU*up -> h slice (in XCD)
//   E  this block's rows of down over the slice's columns     -> down partial (all XCDs)
//      all-reduce as after C                                  -> x
//
// then the final RMSNorm, the output projection (rows split over all blocks)
// with a per-block argmax, and the greedy pick every block reduces itself.
// Before each wait a block stages the weights of its next GEMV (and RMSNorm
// gains) into LDS, so weight traffic overlaps the exchanges. Every wait is
// bounded in time; a block that times out raises the abort flag and every
// block leaves, so the grid always drains.
#include "xdecode.h"

#include "device_util.h"

namespace th {
namespace {

typedef unsigned long long u64;

constexpr int NT = 512;              // threads per block
constexpr int NW = NT / 64;          // waves per block
constexpr int NB = kXBlocksPerXcd;   // blocks per XCD
// Waves 0..NPW-1 poll exchange words and issue no other memory operation
// (vmcnt retires in order, so a poll behind a staging load or a store would
// wait for it); waves NPW.. stage weights and publish results.
constexpr int NPW = 4;
constexpr int NPT = NPW * 64;        // polling threads
constexpr int NWT = NT - NPT;        // worker threads
constexpr int HD = 128;              // head_dim
constexpr int STAGE = 5120;          // 16-byte chunks staged in LDS (80 KB)
constexpr int MAXH = 2560;           // longest vector a block keeps (hidden, MLP slice)
constexpr int MAXRES = 640;          // rows of one block in one phase (output projection: vocab / blocks)
constexpr int RB = 2;                // rows per wave in flight in a streamed GEMV
constexpr int KVROWS = 64;           // cached positions per attention pass
constexpr int MRG = 8192;            // floats of attention partials a block merges
constexpr int TRACE_POINTS = 4;
constexpr int TRACE_SLOTS = 5 * 40 + 2;

template <int G>
struct Shared {
    float x[MAXH];                 // the residual stream
    float in[MAXH];                // the current GEMV's input
    uint4 stage[STAGE];            // staged weights, or the K then V rows of an attention pass
    float res[MAXRES];             // output projection results
    float mrg[MRG];                // attention partials (C), partial sums (all-reduce), PV reduction (B)
    uint16_t gain[MAXH];           // staged RMSNorm gains
    uint16_t qk_gain[2 * HD];      // q_norm then k_norm
    float rope[HD];                // (cos, sin) pairs of the step's position
    float hqkv[(G + 2) * HD];      // the group's q heads, k, v
    float scores[G][KVROWS];
    float st_m[G], st_l[G], st_a[G];
    float wred[NW];
    u64 wred64[NW];
    unsigned ticks[TRACE_SLOTS * TRACE_POINTS];
};

__device__ __forceinline__ unsigned xcc_id() {
    unsigned v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return v & 0xf;
}

__device__ __forceinline__ void dma16(const void *src, void *lds_wave_base) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds_wave_base, 16, 0, 0);
}

// The wave's index within the block, as a scalar.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

__device__ __forceinline__ u64 pack(float v, unsigned epoch) { return ((u64)epoch << 32) | (u64)__float_as_uint(v); }

// Words shared inside an XCD: the store stays in the XCD's L2, the load skips
// the CU's L1. Words shared across XCDs: agent scope both ways.
__device__ __forceinline__ void put_local(u64 *p, float v, unsigned e) {
    __hip_atomic_store(p, pack(v, e), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void put_cross(u64 *p, float v, unsigned e) {
    __hip_atomic_store(p, pack(v, e), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <bool CROSS>
__device__ __forceinline__ u64 get_word(const u64 *p) {
    return CROSS ? __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                 : __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ bool aborted(const XDecodeParams &p) {
    return __hip_atomic_load(p.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

__device__ __forceinline__ void raise_abort(const XDecodeParams &p, int which) {
    if (which) __hip_atomic_fetch_add(p.status + which, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_fetch_add(p.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Polls nseg segments of seg words (segment k at src + k * stride) until every
// word carries `epoch`; word (k, i) lands in dst[k * seg + i]. A thread issues
// the loads of all its missing words (in batches of 8) before examining any,
// so a round costs one round trip. Returns false (block-uniformly) on timeout,
// abort, or a word from a later epoch (a protocol error).
template <bool CROSS>
__device__ __forceinline__ bool wait_words(const XDecodeParams &p, const u64 *src, int seg, int nseg, long long stride, unsigned epoch,
                           float *dst) {
    constexpr int KMAX = 32, KB = 8;
    const int tid = threadIdx.x, n = seg * nseg;
    const bool poller = tid < NPT;
    const long long t0 = (long long)__builtin_amdgcn_s_memrealtime();
    unsigned done = 0;
    for (int it = 0;; ++it) {
        int ok = 1, bad = 0;
#pragma unroll 1
        for (int kb = 0; poller && kb < KMAX && tid + kb * NPT < n; kb += KB) {
            u64 w[KB];
#pragma unroll
            for (int b = 0; b < KB; ++b) {
                const int k = kb + b, i = tid + k * NPT;
                if (i < n && !(done & (1u << k))) {
                    const int sg = i / seg;
                    w[b] = get_word<CROSS>(src + sg * stride + (i - sg * seg));
                }
            }
#pragma unroll
            for (int b = 0; b < KB; ++b) {
                const int k = kb + b, i = tid + k * NPT;
                if (i < n && !(done & (1u << k))) {
                    const int d = (int)((unsigned)(w[b] >> 32) - epoch);
                    if (d == 0) {
                        dst[i] = __uint_as_float((unsigned)w[b]);
                        done |= 1u << k;
                    } else {
                        ok = 0;
                        if (d > 0) bad = 1;
                    }
                }
            }
        }
        int stop = 0;
        if (tid == 0 && (it & 15) == 15) {
            if (aborted(p)) {
                stop = 1;
            } else if ((long long)__builtin_amdgcn_s_memrealtime() - t0 > p.timeout_ticks) {
                stop = 1;
                raise_abort(p, 0);
            }
        }
        if (bad) raise_abort(p, 1);
        if (__syncthreads_and(ok)) return true;
        if (__syncthreads_or(bad || stop)) return false;
    }
}

// Rows of a GEMV phase: up to three runs of rows of row-major bf16 matrices,
// `stride` elements apart, each row read from `cpr` 16-byte chunks.
struct Rows {
    const uint16_t *b0, *b1, *b2;
    int n0, n1;
    int stride, cpr, total;
};

// The row's address as b0 plus an element offset chosen arithmetically (the
// three runs are separate matrices; r differs per lane).
__device__ __forceinline__ const uint16_t *row_at(const Rows &m, int r) {
    const long long d1 = m.b1 - m.b0, d2 = m.b2 - m.b0;
    const bool in0 = r < m.n0, in1 = r < m.n0 + m.n1;
    const long long base = in0 ? 0ll : (in1 ? d1 : d2);
    const int rl = in0 ? r : (in1 ? r - m.n0 : r - m.n0 - m.n1);
    return m.b0 + base + (long long)rl * m.stride;
}

// Chunk f of the block's rows (row-major) sits in stage[f] for f < staged.
__device__ __forceinline__ int staged_chunks(const Rows &m) {
    const int n = m.total * m.cpr;
    return n < STAGE ? n : STAGE;
}

// Issued by the worker waves only.
__device__ __forceinline__ void stage_rows(uint4 *stage, const Rows &m) {
    const int wave = wave_id() - NPW, lane = threadIdx.x & 63;
    if (wave < 0) return;
    const int staged = staged_chunks(m);
    for (int q = wave; q * 64 < staged; q += NW - NPW) {
        const int f = q * 64 + lane;
        if (f < staged) {
            const int r = f / m.cpr, c = f - r * m.cpr;
            dma16(row_at(m, r) + c * 8, stage + q * 64);
        }
    }
}

// Copies `bytes` (a multiple of 16) into LDS through the DMA path (worker waves).
__device__ __forceinline__ void stage_small(const void *src, void *dst, int bytes) {
    const int wave = wave_id() - NPW, lane = threadIdx.x & 63;
    if (wave < 0) return;
    const int chunks = bytes >> 4;
    for (int c0 = wave * 64; c0 < chunks; c0 += (NW - NPW) * 64)
        if (c0 + lane < chunks)
            dma16(reinterpret_cast<const uint4 *>(src) + c0 + lane, reinterpret_cast<uint4 *>(dst) + c0);
}

__device__ __forceinline__ void stage_ready() {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
}

__device__ __forceinline__ float dot8(const uint4 &w, const float *x) {
    const float4 a = reinterpret_cast<const float4 *>(x)[0], b = reinterpret_cast<const float4 *>(x)[1];
    float wf[8];
    unpack8(w, wf);
    float acc = wf[0] * a.x;
    acc = fmaf(wf[1], a.y, acc);
    acc = fmaf(wf[2], a.z, acc);
    acc = fmaf(wf[3], a.w, acc);
    acc = fmaf(wf[4], b.x, acc);
    acc = fmaf(wf[5], b.y, acc);
    acc = fmaf(wf[6], b.z, acc);
    acc = fmaf(wf[7], b.w, acc);
    return acc;
}

// Dot products of up to RB rows (rows[b] < 0: none) with `in`, every chunk of
// every row requested before any is used; staged chunks come from LDS. A row
// has at most 64 CPL chunks.
template <int CPL, int R = RB>
__device__ __forceinline__ void dot_rows(const uint4 *stage, int staged, const Rows &m, const int rows[R],
                                         const float *in, float out[R]) {
    const int lane = threadIdx.x & 63;
    uint4 w[R][CPL];
    static_assert(R * CPL <= 12, "weights in flight per lane bound the registers");
#pragma unroll
    for (int b = 0; b < R; ++b)
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = lane + 64 * i;
            if (rows[b] >= 0 && c < m.cpr) {
                const int f = rows[b] * m.cpr + c;
                w[b][i] = f < staged ? stage[f] : *reinterpret_cast<const uint4 *>(row_at(m, rows[b]) + c * 8);
            }
        }
#pragma unroll
    for (int b = 0; b < R; ++b) {
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = lane + 64 * i;
            if (rows[b] >= 0 && c < m.cpr) acc += dot8(w[b][i], in + c * 8);
        }
        out[b] = wave_sum_dpp(acc);
    }
}

// in = x * gain (staged), returns 1 / sqrt(mean(x^2) + eps) (model/cpu.rs:85-94
// with the scale applied after the dot products). Ends with a barrier.
template <int G>
__device__ __forceinline__ float norm_input(Shared<G> &sh, int H, float eps) {
    const int tid = threadIdx.x;
    float ss = 0.f;
    for (int i = tid; i < H; i += NT) {
        const float v = sh.x[i];
        ss += v * v;
        sh.in[i] = v * bf16_to_f32(sh.gain[i]);
    }
    ss = wave_sum_dpp(ss);
    if ((tid & 63) == 0) sh.wred[wave_id()] = ss;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) t += sh.wred[w];
    return 1.0f / sqrtf(t / (float)H + eps);
}

template <int G>
__device__ __forceinline__ void trace_at(Shared<G> &sh, const XDecodeParams &p, int s, int slot, int which) {
    if (p.trace && blockIdx.x == 0 && threadIdx.x == 0 && s < p.trace_steps && slot < TRACE_SLOTS)
        sh.ticks[slot * TRACE_POINTS + which] = (unsigned)__builtin_amdgcn_s_memrealtime();
}

template <int G>
__device__ __forceinline__ void trace_flush(Shared<G> &sh, const XDecodeParams &p, int s) {
    if (!p.trace || blockIdx.x != 0 || s >= p.trace_steps) return;
    __syncthreads();
    const int words = (p.n_layers * 5 + 2) * TRACE_POINTS;
    for (int i = threadIdx.x; i < words; i += NT)
        p.trace[1 + (size_t)s * words + i] = i < TRACE_SLOTS * TRACE_POINTS ? sh.ticks[i] : 0;
    __syncthreads();
    for (int i = threadIdx.x; i < TRACE_SLOTS * TRACE_POINTS; i += NT) sh.ticks[i] = 0;
}

__device__ __forceinline__ void load_row8(const float *row, int sub, float f[8]) {
    const float4 a = reinterpret_cast<const float4 *>(row)[sub * 2], b = reinterpret_cast<const float4 *>(row)[sub * 2 + 1];
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}
__device__ __forceinline__ void load_row8(const uint16_t *row, int sub, float f[8]) {
    unpack8(reinterpret_cast<const uint4 *>(row)[sub], f);
}
__device__ __forceinline__ float load_at(const float *row, int d) { return row[d]; }
__device__ __forceinline__ float load_at(const uint16_t *row, int d) { return bf16_to_f32(row[d]); }

// Positions per attention split: a multiple of 16, at least 32, and few
// enough splits that their partials fit the merge buffer and the XCD's blocks.
// Short splits spread the cache reads of a head over several CUs.
template <int G>
__device__ __forceinline__ long long split_chunk(long long len) {
    constexpr int maxs = (MRG / (G * (HD + 2))) < NB ? (MRG / (G * (HD + 2))) : NB;
    long long c = (len + maxs - 1) / maxs;
    c = (c + 15) / 16 * 16;
    return c < 32 ? 32 : c;
}

// Phase B for split j of the group's positions 0..pos: stages the first pass of
// cached rows, waits for the group's q/k/v, RMSNorms and rotates them,
// attends, appends the new key and value, and publishes (acc, m, l).
template <int G, typename KV>
__device__ __forceinline__ bool attention(Shared<G> &sh, const XDecodeParams &p, int layer, int g, int j, long long pos,
                          unsigned e_qkv, unsigned e_att, const LayerWeights &W) {
    constexpr int LPK = HD / 8, KPW = 64 / LPK, KPB = NW * KPW, NP = NT / HD, HALF = HD / 2;
    constexpr int ROW16 = HD * (int)sizeof(KV) / 16;
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id(), sub = lane % LPK;
    const long long len = pos + 1, chunk = split_chunk<G>(len);
    const long long s0 = (long long)j * chunk, s1 = s0 + chunk < len ? s0 + chunk : len;
    const size_t per = (size_t)p.n_kv_heads * p.max_len * HD;
    KV *kc = reinterpret_cast<KV *>(p.kv) + (size_t)(layer * 2 + 0) * per + (size_t)g * p.max_len * HD;
    KV *vc = reinterpret_cast<KV *>(p.kv) + (size_t)(layer * 2 + 1) * per + (size_t)g * p.max_len * HD;
    uint4 *kst = sh.stage, *vst = sh.stage + KVROWS * ROW16;
    auto cached_in = [&](long long c0, int cnt) -> int {
        const long long nc = pos - c0;
        return nc <= 0 ? 0 : (nc < cnt ? (int)nc : cnt);
    };
    auto stage_kv = [&](long long c0, int ncache) {
        const int chunks = ncache * ROW16;
        const uint4 *ks = reinterpret_cast<const uint4 *>(kc + c0 * HD);
        const uint4 *vs = reinterpret_cast<const uint4 *>(vc + c0 * HD);
        if (wave < NPW) return;
        for (int base = (wave - NPW) * 64; base < chunks; base += NWT)
            if (base + lane < chunks) {
                dma16(ks + base + lane, kst + base);
                dma16(vs + base + lane, vst + base);
            }
    };
    {
        const int cnt0 = (int)(s1 - s0 < KVROWS ? s1 - s0 : KVROWS);
        stage_kv(s0, cached_in(s0, cnt0));
    }
    if (W.q_norm) stage_small(W.q_norm, sh.qk_gain, HD * 2);
    if (W.k_norm) stage_small(W.k_norm, sh.qk_gain + HD, HD * 2);
    stage_small(p.rope + pos * HD, sh.rope, HD * 4);
    if (tid < G) {
        sh.st_m[tid] = -INFINITY;
        sh.st_l[tid] = 0.f;
    }
    if (!wait_words<false>(p, p.qkv_loc + (size_t)g * (G + 2) * HD, (G + 2) * HD, 1, 0, e_qkv, sh.hqkv)) return false;
    stage_ready();
    // q/k RMSNorm (model.rs:111-116) and RoPE (model.rs:117-118), one wave per head.
    for (int h = wave; h <= G; h += NW) {
        float *x = sh.hqkv + h * HD;
        const bool has_gain = h < G ? W.q_norm != nullptr : W.k_norm != nullptr;
        const uint16_t *gain = sh.qk_gain + (h < G ? 0 : HD);
        float a = x[lane], b = x[lane + HALF];
        if (has_gain) {
            const float ss = wave_sum_dpp(a * a + b * b);
            const float sc = 1.0f / sqrtf(ss / (float)HD + p.eps);
            a = a * (sc * bf16_to_f32(gain[lane]));
            b = b * (sc * bf16_to_f32(gain[lane + HALF]));
        }
        const float c = sh.rope[2 * lane], s = sh.rope[2 * lane + 1];
        x[lane] = a * c - b * s;
        x[lane + HALF] = b * c + a * s;
    }
    __syncthreads();
    const float *hk = sh.hqkv + G * HD, *hv = sh.hqkv + (G + 1) * HD;
    float qf[G][8];
#pragma unroll
    for (int gg = 0; gg < G; ++gg)
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[gg][i] = sh.hqkv[gg * HD + sub * 8 + i];
    const float scale = 1.0f / sqrtf((float)HD);
    const int d = tid % HD, pt = tid / HD;
    const KV *ks_l = reinterpret_cast<const KV *>(kst), *vs_l = reinterpret_cast<const KV *>(vst);
    float acc[G];
#pragma unroll
    for (int gg = 0; gg < G; ++gg) acc[gg] = 0.f;
    for (long long c0 = s0; c0 < s1; c0 += KVROWS) {
        const int cnt = (int)(s1 - c0 < KVROWS ? s1 - c0 : KVROWS);
        const int ncache = cached_in(c0, cnt);
        if (c0 != s0) {
            stage_kv(c0, ncache);
            stage_ready();
        }
        for (int j0 = 0; j0 < cnt; j0 += KPB) {
            const int jj = j0 + wave * KPW + lane / LPK;
            float kf[8];
            if (jj < ncache) {
                load_row8(ks_l + jj * HD, sub, kf);
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) kf[i] = jj < cnt ? hk[sub * 8 + i] : 0.f;
            }
#pragma unroll
            for (int gg = 0; gg < G; ++gg) {
                float sc = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) sc = fmaf(qf[gg][i], kf[i], sc);
                sc = group_sum<LPK>(sc);
                if (jj < cnt && sub == 0) sh.scores[gg][jj] = scale * sc;
            }
        }
        __syncthreads();
        for (int gg = wave; gg < G; gg += NW) {
            float m = -INFINITY;
            for (int t = lane; t < cnt; t += 64) m = fmaxf(m, sh.scores[gg][t]);
            m = wave_max(m);
            const float m_old = sh.st_m[gg], m_new = fmaxf(m_old, m);
            float l = 0.f;
            for (int t = lane; t < cnt; t += 64) {
                const float e = expf(sh.scores[gg][t] - m_new);
                sh.scores[gg][t] = e;
                l += e;
            }
            l = wave_sum_dpp(l);
            if (lane == 0) {
                const float al = expf(m_old - m_new);
                sh.st_a[gg] = al;
                sh.st_l[gg] = sh.st_l[gg] * al + l;
                sh.st_m[gg] = m_new;
            }
        }
        __syncthreads();
#pragma unroll
        for (int gg = 0; gg < G; ++gg) acc[gg] *= sh.st_a[gg];
        for (int t = pt; t < cnt; t += NP) {
            const float v = t < ncache ? load_at(vs_l + t * HD, d) : hv[d];
#pragma unroll
            for (int gg = 0; gg < G; ++gg) acc[gg] = fmaf(sh.scores[gg][t], v, acc[gg]);
        }
        __syncthreads();  // the stage and scores are rewritten by the next pass
    }
    // The split holding pos appends the new key and value (model.rs:119-120);
    // the stores complete before the block goes on, so a later step's reader on
    // this XCD finds them in its L2.
    const int wt = tid - NPT;  // worker thread index (negative on polling waves)
    if (pos >= s0 && pos < s1 && wt >= 0 && wt < HD) {
        store_kv(kc + pos * HD + wt, hk[wt]);
        store_kv(vc + pos * HD + wt, hv[wt]);
    }
#pragma unroll
    for (int gg = 0; gg < G; ++gg) sh.mrg[gg * NT + tid] = acc[gg];
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    u64 *out = p.att_loc + ((size_t)g * NB + j) * G * (HD + 2);
    for (int i = wt; wt >= 0 && i < G * (HD + 2); i += NWT) {
        const int gg = i / (HD + 2), dd = i - gg * (HD + 2);
        float v;
        if (dd < HD) {
            v = sh.mrg[gg * NT + dd];
#pragma unroll
            for (int q = 1; q < NP; ++q) v += sh.mrg[gg * NT + q * HD + dd];
        } else {
            v = dd == HD ? sh.st_m[gg] : sh.st_l[gg];
        }
        put_local(out + i, v, e_att);
    }
    return true;
}

// Phase C's input: the group's attention output merged from its splits' (acc, m, l).
template <int G>
__device__ __forceinline__ void merge_attention(Shared<G> &sh, int nsplit) {
    for (int t = threadIdx.x; t < G * HD; t += NT) {
        const int gg = t / HD, dd = t - gg * HD;
        float m = -INFINITY;
        for (int s = 0; s < nsplit; ++s) m = fmaxf(m, sh.mrg[(s * G + gg) * (HD + 2) + HD]);
        float l = 0.f, a = 0.f;
        for (int s = 0; s < nsplit; ++s) {
            const float *slot = sh.mrg + (s * G + gg) * (HD + 2);
            const float ms = slot[HD];
            if (ms != -INFINITY) {
                const float w = expf(ms - m);
                l += slot[HD + 1] * w;
                a += slot[dd] * w;
            }
        }
        sh.in[t] = a / l;
    }
    __syncthreads();
}

// The all-reduce after o or down: the eight XCDs' partial sums of this block's
// residual rows, added to x in XCD order, shared inside the XCD, then every
// block gathers all of x.
template <int G>
__device__ __forceinline__ bool all_reduce(Shared<G> &sh, const XDecodeParams &p, const u64 *part, int g, int r0,
                                           int nr, unsigned e_part, unsigned e_x) {
    const int H = p.hidden, tid = threadIdx.x;
    if (!wait_words<true>(p, part + r0, nr, kXcds, H, e_part, sh.mrg)) return false;
    const int wt = tid - NPT;
    if (wt >= 0 && wt < nr) {
        float v = sh.x[r0 + wt];
        float o = 0.f;
#pragma unroll
        for (int k = 0; k < kXcds; ++k) o += sh.mrg[k * nr + wt];
        put_local(p.x_loc + (size_t)g * H + r0 + wt, v + o, e_x);
    }
    return wait_words<false>(p, p.x_loc + (size_t)g * H, H, 1, 0, e_x, sh.x);
}

// CPLH: 16-byte chunks per lane of a hidden-wide row (q/k/v, gate/up, output
// projection); CPLO, CPLD: of a row of o over the group's columns and of down
// over the MLP slice's columns.
template <int G, int CPLH, int CPLD>
__global__ __launch_bounds__(NT) void xdecode_kernel(XDecodeParams p) {
    constexpr int CPLO = (G * HD / 8 + 63) / 64;
    __shared__ Shared<G> sh;
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id(), blk = blockIdx.x, nblk = gridDim.x;
    const int g = blk % kXcds, j = blk / kXcds;
    // Every block checks that it runs on the XCD its index implies.
    if (xcc_id() != (unsigned)g) {
        if (tid == 0) raise_abort(p, 2);
        return;
    }
    const int H = p.hidden, I = p.intermediate, L = p.n_layers, V = p.vocab;
    const int qd = p.n_heads * HD, IS = I / kXcds, RA = (G + 2) * HD;
    // This block's rows: q/k/v of the group, residual rows, MLP pairs, output projection rows.
    const int a0 = j * RA / NB, na = RA / NB;
    const int r0 = j * H / NB, nr = H / NB;
    const int p0 = j * IS / NB, np = IS / NB;
    const int v0 = (int)((long long)blk * V / nblk), nv = (int)((long long)(blk + 1) * V / nblk) - v0;
    const unsigned EPS = xdecode_epochs_per_step(L);

    StepState *st = p.step;
    const long long pos0 = st->pos, step0 = st->step;
    unsigned token = st->token;
    float *const keep = st->logits_out;
    if (p.trace && blk == 0 && tid == 0) p.trace[0] = __builtin_amdgcn_s_memrealtime() & 0xffffffffull;
    for (int i = tid; i < TRACE_SLOTS * TRACE_POINTS; i += NT) sh.ticks[i] = 0;

    auto qkv_rows = [&](const LayerWeights &W) {
        Rows m;
        // The group's rows in exchange order: its q heads, its k head, its v head.
        const int qa = a0 < G * HD ? a0 : G * HD, qb = a0 + na < G * HD ? a0 + na : G * HD;
        const int ka = a0 < G * HD ? 0 : (a0 < (G + 1) * HD ? a0 - G * HD : HD);
        const int kb = a0 + na <= G * HD ? 0 : (a0 + na < (G + 1) * HD ? a0 + na - G * HD : HD);
        const int va = a0 <= (G + 1) * HD ? 0 : a0 - (G + 1) * HD;
        m.b0 = W.q + ((size_t)g * G * HD + qa) * H;
        m.n0 = qb - qa;
        m.b1 = W.k + ((size_t)g * HD + ka) * H;
        m.n1 = kb - ka;
        m.b2 = W.v + ((size_t)g * HD + va) * H;
        m.stride = H;
        m.cpr = H / 8;
        m.total = na;
        return m;
    };
    auto o_rows = [&](const LayerWeights &W) {
        Rows m;
        m.b0 = W.o + (size_t)r0 * qd + (size_t)g * G * HD;
        m.n0 = nr;
        m.n1 = 0;
        m.b1 = m.b2 = m.b0;
        m.stride = qd;
        m.cpr = G * HD / 8;
        m.total = nr;
        return m;
    };
    auto mlp_rows = [&](const LayerWeights &W) {
        Rows m;
        m.b0 = W.gate + ((size_t)g * IS + p0) * H;
        m.n0 = np;
        m.b1 = W.up + ((size_t)g * IS + p0) * H;
        m.n1 = np;
        m.b2 = m.b1;
        m.stride = H;
        m.cpr = H / 8;
        m.total = 2 * np;
        return m;
    };
    auto down_rows = [&](const LayerWeights &W) {
        Rows m;
        m.b0 = W.down + (size_t)r0 * I + (size_t)g * IS;
        m.n0 = nr;
        m.n1 = 0;
        m.b1 = m.b2 = m.b0;
        m.stride = I;
        m.cpr = IS / 8;
        m.total = nr;
        return m;
    };
    auto head_rows = [&]() {
        Rows m;
        m.b0 = p.lm_head + (size_t)v0 * H;
        m.n0 = nv;
        m.n1 = 0;
        m.b1 = m.b2 = m.b0;
        m.stride = H;
        m.cpr = H / 8;
        m.total = nv;
        return m;
    };

    // The first layer's q/k/v weights and gains, before the loop.
    stage_rows(sh.stage, qkv_rows(p.layers[0]));
    stage_small(p.layers[0].attn_norm, sh.gain, H * 2);

    for (int s = 0; s < p.steps; ++s) {
        const long long pos = pos0 + s;
        const unsigned eb = p.epoch_base + (unsigned)s * EPS;
        // The token's embedding row (model/cpu.rs:38-47) is every block's x.
        {
            const uint4 *row = reinterpret_cast<const uint4 *>(p.embed + (size_t)token * H);
            for (int c = tid; c < H / 8; c += NT) {
                float f[8];
                unpack8(row[c], f);
#pragma unroll
                for (int e8 = 0; e8 < 8; ++e8) sh.x[c * 8 + e8] = f[e8];
            }
        }
        const long long len = pos + 1;
        const int nsplit = (int)((len + split_chunk<G>(len) - 1) / split_chunk<G>(len));
        for (int l = 0; l < L; ++l) {
            const LayerWeights &W = p.layers[l];
            const unsigned e = eb + (unsigned)l * 7;
            // ---- A: attention RMSNorm, q/k/v rows -> qkv (in XCD)
            const int ph = l * 5;
            trace_at(sh, p, s, ph, 0);
            stage_ready();
            {
                const Rows m = qkv_rows(W);
                const int staged = staged_chunks(m);
                const float sc = norm_input(sh, H, p.eps);
                for (int q0 = wave; q0 < m.total; q0 += NW * RB) {
                    int rows[RB];
                    float out[RB];
#pragma unroll
                    for (int b = 0; b < RB; ++b) rows[b] = q0 + b * NW < m.total ? q0 + b * NW : -1;
                    dot_rows<CPLH>(sh.stage, staged, m, rows, sh.in, out);
                    if (lane == 0)
#pragma unroll
                        for (int b = 0; b < RB; ++b)
                            if (rows[b] >= 0) sh.res[rows[b]] = sc * out[b];
                }
            }
            __syncthreads();  // results are in res; the stage is rewritten next
            for (int i = tid - NPT; i >= 0 && i < na; i += NWT)
                put_local(p.qkv_loc + (size_t)g * RA + a0 + i, sh.res[i], e + 1);
            trace_at(sh, p, s, ph, 3);
            // ---- B: attention (blocks 0..nsplit-1 of the XCD)
            trace_at(sh, p, s, ph + 1, 0);
            if (j < nsplit) {
                const bool ok = p.kv_bf16 ? attention<G, uint16_t>(sh, p, l, g, j, pos, e + 1, e + 2, W)
                                          : attention<G, float>(sh, p, l, g, j, pos, e + 1, e + 2, W);
                if (!ok) return;
                __syncthreads();
            }
            trace_at(sh, p, s, ph + 1, 3);
            // ---- C: o rows over the group's columns -> partial; all-reduce -> x
            {
                const Rows m = o_rows(W);
                stage_rows(sh.stage, m);
                if (!wait_words<false>(p, p.att_loc + (size_t)g * NB * G * (HD + 2), G * (HD + 2), nsplit,
                                       (long long)G * (HD + 2), e + 2, sh.mrg))
                    return;
                trace_at(sh, p, s, ph + 2, 0);
                stage_ready();
                merge_attention(sh, nsplit);
                const int staged = staged_chunks(m);
                for (int q0 = wave; q0 < m.total; q0 += NW * RB) {
                    int rows[RB];
                    float out[RB];
#pragma unroll
                    for (int b = 0; b < RB; ++b) rows[b] = q0 + b * NW < m.total ? q0 + b * NW : -1;
                    dot_rows<CPLO>(sh.stage, staged, m, rows, sh.in, out);
                    if (lane == 0)
#pragma unroll
                        for (int b = 0; b < RB; ++b)
                            if (rows[b] >= 0) sh.res[rows[b]] = out[b];
                }
                __syncthreads();  // results are in res; the stage is rewritten next
                for (int i = tid - NPT; i >= 0 && i < nr; i += NWT)
                    put_cross(p.part + (size_t)g * H + r0 + i, sh.res[i], e + 3);
                stage_rows(sh.stage, mlp_rows(W));
                stage_small(W.mlp_norm, sh.gain, H * 2);
                if (!all_reduce(sh, p, p.part, g, r0, nr, e + 3, e + 4)) return;
                trace_at(sh, p, s, ph + 2, 3);
            }
            // ---- D: MLP RMSNorm, gate/up pairs, SiLU * up -> h slice (in XCD)
            {
                trace_at(sh, p, s, ph + 3, 0);
                stage_ready();
                const Rows m = mlp_rows(W);
                const int staged = staged_chunks(m);
                const float sc = norm_input(sh, H, p.eps);
                for (int q0 = wave; q0 < np; q0 += NW * (RB / 2)) {
                    int rows[RB];
                    float out[RB];
#pragma unroll
                    for (int b = 0; b < RB / 2; ++b) {
                        const int pr = q0 + b * NW;
                        rows[2 * b] = pr < np ? pr : -1;
                        rows[2 * b + 1] = pr < np ? np + pr : -1;
                    }
                    dot_rows<CPLH>(sh.stage, staged, m, rows, sh.in, out);
                    if (lane == 0)
#pragma unroll
                        for (int b = 0; b < RB / 2; ++b)
                            if (rows[2 * b] >= 0) {
                                const float gt = sc * out[2 * b], up = sc * out[2 * b + 1];
                                sh.res[rows[2 * b]] = silu(gt) * up;
                            }
                }
                __syncthreads();  // results are in res; the stage is rewritten next
                for (int i = tid - NPT; i >= 0 && i < np; i += NWT)
                    put_local(p.h_loc + (size_t)g * IS + p0 + i, sh.res[i], e + 5);
                trace_at(sh, p, s, ph + 3, 3);
            }
            // ---- E: down rows over the slice's columns -> partial; all-reduce -> x
            {
                trace_at(sh, p, s, ph + 4, 0);
                const Rows m = down_rows(W);
                stage_rows(sh.stage, m);
                if (!wait_words<false>(p, p.h_loc + (size_t)g * IS, IS, 1, 0, e + 5, sh.in)) return;
                stage_ready();
                const int staged = staged_chunks(m);
                for (int q0 = wave; q0 < m.total; q0 += NW * RB) {
                    int rows[RB];
                    float out[RB];
#pragma unroll
                    for (int b = 0; b < RB; ++b) rows[b] = q0 + b * NW < m.total ? q0 + b * NW : -1;
                    dot_rows<CPLD>(sh.stage, staged, m, rows, sh.in, out);
                    if (lane == 0)
#pragma unroll
                        for (int b = 0; b < RB; ++b)
                            if (rows[b] >= 0) sh.res[rows[b]] = out[b];
                }
                __syncthreads();  // results are in res; the stage is rewritten next
                for (int i = tid - NPT; i >= 0 && i < nr; i += NWT)
                    put_cross(p.part + (size_t)kXcds * H + (size_t)g * H + r0 + i, sh.res[i], e + 6);
                if (l + 1 < L) {
                    stage_rows(sh.stage, qkv_rows(p.layers[l + 1]));
                    stage_small(p.layers[l + 1].attn_norm, sh.gain, H * 2);
                } else {
                    stage_rows(sh.stage, head_rows());
                    stage_small(p.norm, sh.gain, H * 2);
                }
                if (!all_reduce(sh, p, p.part + (size_t)kXcds * H, g, r0, nr, e + 6, e + 7)) return;
                trace_at(sh, p, s, ph + 4, 3);
            }
        }
        // ---- the final RMSNorm, the output projection and this block's argmax
        const int phf = L * 5;
        trace_at(sh, p, s, phf, 0);
        stage_ready();
        uint64_t best = 0;
        {
            const Rows m = head_rows();
            const int staged = staged_chunks(m);
            const float sc = norm_input(sh, H, p.eps);
            constexpr int RH = 12 / CPLH;  // output-projection rows per wave in flight
            for (int q0 = wave; q0 < m.total; q0 += NW * RH) {
                int rows[RH];
                float out[RH];
#pragma unroll
                for (int b = 0; b < RH; ++b) rows[b] = q0 + b * NW < m.total ? q0 + b * NW : -1;
                dot_rows<CPLH, RH>(sh.stage, staged, m, rows, sh.in, out);
#pragma unroll
                for (int b = 0; b < RH; ++b)
                    if (rows[b] >= 0) {
                        const float lg = sc * out[b];
                        if (lane == 0) sh.res[rows[b]] = lg;
                        best = max_u64(best, argmax_pack(lg, (uint32_t)(v0 + rows[b])));
                    }
            }
        }
        if (lane == 0) sh.wred64[wave] = best;
        __syncthreads();
        const unsigned e_am = eb + (unsigned)L * 7 + 1;
        for (int i = tid - NPT; i >= 0 && i < nv; i += NWT) {
            p.logits[v0 + i] = sh.res[i];
            if (keep) keep[(size_t)(step0 + s) * V + v0 + i] = sh.res[i];
        }
        if (tid == NPT) {
            uint64_t b = 0;
            for (int w = 0; w < NW; ++w) b = max_u64(b, sh.wred64[w]);
            u64 *am = p.am + (size_t)blk * 2;
            __hip_atomic_store(am, ((u64)e_am << 32) | (b >> 32), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(am + 1, ((u64)e_am << 32) | (b & 0xffffffffull), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
        trace_at(sh, p, s, phf, 3);
        __syncthreads();  // the stage is rewritten next
        // The next step's first weights, then the greedy pick every block reduces.
        stage_rows(sh.stage, qkv_rows(p.layers[0]));
        stage_small(p.layers[0].attn_norm, sh.gain, H * 2);
        if (!wait_words<true>(p, p.am, 2 * nblk, 1, 0, e_am, sh.mrg)) return;
        trace_at(sh, p, s, phf + 1, 0);
        {
            uint64_t b = 0;
            for (int i = tid; i < nblk; i += NT)
                b = max_u64(b, ((uint64_t)__float_as_uint(sh.mrg[2 * i]) << 32) | __float_as_uint(sh.mrg[2 * i + 1]));
            b = wave_max_u64(b);
            if (lane == 0) sh.wred64[wave] = b;
            __syncthreads();
            b = 0;
            for (int w = 0; w < NW; ++w) b = max_u64(b, sh.wred64[w]);
            token = argmax_index(b);
        }
        if (blk == 0 && tid == 0 && st->tokens_out) st->tokens_out[step0 + s + 1] = token;
        trace_at(sh, p, s, phf + 1, 3);
        trace_flush(sh, p, s);
        __syncthreads();  // wred64 and x are rewritten next
    }
    if (blk == 0 && tid == 0) {
        st->pos = pos0 + p.steps;
        st->step = step0 + p.steps;
        st->token = token;
    }
}

}  // namespace

// The (chunks per lane) shapes compiled: a 1024-wide model with an MLP slice of
// up to 512 columns (Qwen3-0.6B), and a 2560-wide one with slices of up to 1536
// (Qwen3-4B).
bool xdecode_shape(int hidden, int intermediate, int &cplh, int &cpld) {
    const int h = (hidden / 8 + 63) / 64, d = (intermediate / kXcds / 8 + 63) / 64;
    if (h <= 2 && d <= 1) { cplh = 2; cpld = 1; return true; }
    if (h <= 5 && d <= 3) { cplh = 5; cpld = 3; return true; }
    return false;
}

// The instances compiled: Qwen3-0.6B's shape (2 query heads per KV head,
// hidden 1024, MLP slice <= 512) and Qwen3-4B's (4, 2560, <= 1536).
const void *xdecode_fn(int g, int cplh, int cpld) {
    if (g == 2 && cplh == 2 && cpld == 1) return (const void *)xdecode_kernel<2, 2, 1>;
    if (g == 4 && cplh == 5 && cpld == 3) return (const void *)xdecode_kernel<4, 5, 3>;
    return nullptr;
}

bool xdecode_supported(int hidden, int intermediate, int n_heads, int n_kv_heads, int head_dim, int vocab, int blocks) {
    if (head_dim != HD || n_kv_heads != kXcds || blocks != kXcds * NB) return false;
    const int g = n_heads % n_kv_heads == 0 ? n_heads / n_kv_heads : 0;
    if (g != 1 && g != 2 && g != 4) return false;
    if (hidden > MAXH || hidden % (8 * NB) != 0 || hidden % 64 != 0) return false;
    const int is = intermediate / kXcds;
    if (intermediate % (kXcds * NB) != 0 || is % 8 != 0 || is > MAXH) return false;
    if (((g + 2) * HD) % NB != 0) return false;
    int cplh, cpld;
    if (!xdecode_shape(hidden, intermediate, cplh, cpld) || !xdecode_fn(g, cplh, cpld)) return false;
    if (vocab <= 0 || (vocab + blocks - 1) / blocks > MAXRES || 2 * blocks > MRG) return false;
    // The merge buffer holds at least one split and an all-reduce's partial sums.
    if (g * (HD + 2) > MRG || kXcds * (hidden / NB) > MRG) return false;
    return true;
}

hipError_t launch_xdecode(hipStream_t s, const XDecodeParams &p, int blocks) {
    if (!xdecode_supported(p.hidden, p.intermediate, p.n_heads, p.n_kv_heads, p.head_dim, p.vocab, blocks))
        return hipErrorInvalidValue;
    XDecodeParams copy = p;
    void *args[] = {&copy};
    int cplh = 0, cpld = 0;
    xdecode_shape(p.hidden, p.intermediate, cplh, cpld);
    const int g = p.n_heads / p.n_kv_heads;
    const void *fn = xdecode_fn(g, cplh, cpld);
    if (!fn) return hipErrorInvalidValue;
    return hipLaunchCooperativeKernel(fn, dim3(blocks), dim3(NT), args, 0, s);
}

}  // namespace th
