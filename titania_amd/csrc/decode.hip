// The persistent decode kernel: every step of a greedy decode (model/chat.rs:149-178
// at temperature 0, each step one pass of model/model.rs:93-149 for one token)
// in one cooperative launch of one block per CU.
//
// Each layer is five phases; between phases, blocks hand vectors to each other
// through exchange buffers of 64-bit words holding (f32 bits, epoch). A
// producer writes each value once with a relaxed device-scope store, copied to
// one replica per XCD; consumers poll their replica until every word carries
// the phase's epoch, so data and its readiness travel together and no fence or
// flag is needed. Before waiting, every block issues the loads of its share of
// the phase's weights, which do not depend on the data being waited for.
//
//   A  attention RMSNorm (each block normalizes the whole residual itself),
//      q/k/v GEMV rows                                 -> exchange qkv
//   B  per KV head: q/k RMSNorm, RoPE, KV append, attention over the cache
//      (split over positions; the last split to finish merges) -> exchange att
//   C  o GEMV rows + residual add on the block's own rows     -> exchange x
//   D  MLP RMSNorm, gate and up rows of the same indices, SiLU * up -> exchange h
//   E  down GEMV rows + residual add                          -> exchange x
// then the final RMSNorm, the output projection with a per-block argmax, and
// the greedy pick that every block reduces for itself.
//
// Every wait is bounded in time; a block that times out raises the abort flag
// and every block leaves, so the grid always drains.
#include "common.h"
#include "decode.h"
#include "device_util.h"

namespace th {

namespace {

constexpr int NT = 512;              // threads per block
constexpr int NW = NT / 64;          // waves per block
constexpr int NPOLL = NW;            // waves that poll exchange buffers (and stage weights before polling)
constexpr int PUB = NW - 1;          // the wave that publishes results (it never polls)
constexpr int STAGE = 4096;          // 16-byte chunks staged in LDS ahead of a wait (64 KB)
constexpr int MAX_COLS = 10240;      // longest input vector kept in LDS (floats)
constexpr int MAX_PART = 4096;       // per-unit partial sums of a GEMV phase
constexpr int MAX_RES = 1024;        // rows one block finishes in one pass
constexpr int MAX_OWN = 16;          // residual rows a block owns
constexpr int MAX_H = 4096;          // longest hidden state (RMSNorm gains staged in LDS)
constexpr int MAXG = 8;              // query heads per KV head
constexpr int MAX_HD = 256;
constexpr int SUB = 256;             // attention positions scored per pass
constexpr int TRACE_POINTS = 4;      // per phase: input ready, staged data ready, computed, published
constexpr int TRACE_SLOTS = 5 * 40 + 2;  // phases of up to 40 layers, output projection, pick

typedef unsigned long long u64;

struct Shared {
    float xin[MAX_COLS];
    float part[MAX_PART];
    float res[MAX_RES];
    float xown[MAX_OWN];
    float hqkv[(MAXG + 2) * MAX_HD];  // one KV group's q heads, then k, then v
    float scores[MAXG][SUB];
    // Weights of the coming GEMV, or cached K then V rows of an attention split,
    // loaded straight into LDS while the block waits for its input.
    uint4 stage[STAGE];
    uint16_t gain[MAX_H];        // the coming RMSNorm's gains
    uint16_t qk_gain[2 * MAX_HD];  // q_norm then k_norm gains of the layer
    float rope_row[MAX_HD];      // (cos, sin) pairs of the step's position
    float st_m[MAXG], st_l[MAXG], st_a[MAXG];
    float red[NW];
    u64 red64[NW];
    int flag;
    unsigned ticks[TRACE_SLOTS * TRACE_POINTS];  // this step's trace (low 32 bits), flushed after the pick
};

__device__ __forceinline__ void lds_dma16(const void *src, uint4 *wave_base) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)wave_base, 16, 0, 0);
}

__device__ __forceinline__ u64 pack(float v, unsigned epoch) {
    return ((u64)epoch << 32) | (u64)__float_as_uint(v);
}

__device__ __forceinline__ void publish(u64 *base, int stride, int i, float v, unsigned epoch, int replicas) {
    const u64 w = pack(v, epoch);
    for (int r = 0; r < replicas; ++r)
        __hip_atomic_store(base + (size_t)r * stride + i, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool aborted(const DecodeParams &p) {
    return __hip_atomic_load(p.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

__device__ __forceinline__ void raise_abort(const DecodeParams &p, int protocol) {
    __hip_atomic_fetch_add(p.status + (protocol ? 1 : 0), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (protocol) __hip_atomic_fetch_add(p.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Polls n exchange words until all carry `epoch`, copying their values to dst
// (LDS). Each round, a thread issues the loads of all its words still missing
// before looking at any, so a round costs one memory round trip. Returns false
// (block-uniformly) on timeout, abort or a word from a later epoch (a protocol
// error).
__device__ __forceinline__ bool wait_vec(const DecodeParams &p, const u64 *src, int n, unsigned epoch, float *dst) {
    constexpr int NP = NPOLL * 64;
    constexpr int KMAX = 24;  // words per thread: n <= KMAX * NP
    constexpr int KB = 8;
    static_assert(KMAX * NP >= MAX_COLS && KMAX <= 32, "poll bitmask must cover the longest vector");
    const int tid = threadIdx.x;
    __syncthreads();  // dst may still be read by the previous phase
    const long long t0 = (long long)__builtin_amdgcn_s_memrealtime();
    unsigned done = 0;  // bit k: word tid + k*NP already taken
    for (int it = 0;; ++it) {
        int ok = 1, bad = 0;
        if (tid < NP) {
            // Batches of KB words: every load of a batch is in flight before
            // the first is examined (one batch covers n <= KB * NP).
#pragma unroll 1
            for (int kb = 0; kb < KMAX; kb += KB) {
                if (tid + kb * NP >= n) break;
                u64 w[KB];
#pragma unroll
                for (int j = 0; j < KB; ++j) {
                    const int k = kb + j, i = tid + k * NP;
                    if (i < n && !(done & (1u << k)))
                        w[j] = __hip_atomic_load(src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
#pragma unroll
                for (int j = 0; j < KB; ++j) {
                    const int k = kb + j, i = tid + k * NP;
                    if (i < n && !(done & (1u << k))) {
                        const int d = (int)((unsigned)(w[j] >> 32) - epoch);
                        if (d == 0) {
                            dst[i] = __uint_as_float((unsigned)w[j]);
                            done |= 1u << k;
                        } else {
                            ok = 0;
                            if (d > 0) bad = 1;
                        }
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

// Block-wide sum (deterministic order), every thread gets it.
__device__ __forceinline__ float block_sum(Shared &sh, float v) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh.red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = 0.f;
    for (int w = 0; w < NW; ++w) s += sh.red[w];
    return s;
}

// xin[0..n) = xin * (1/sqrt(mean square + eps) * gain): model/cpu.rs:85-94 on
// one row, with the gains staged in sh.gain.
__device__ __forceinline__ void rmsnorm_lds(Shared &sh, int n, float eps) {
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += NT) ss += sh.xin[i] * sh.xin[i];
    const float total = block_sum(sh, ss);
    const float scale = 1.0f / sqrtf(total / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += NT) sh.xin[i] = sh.xin[i] * (scale * bf16_to_f32(sh.gain[i]));
    __syncthreads();
}

// A GEMV phase of one block: nrows rows of cpr 16-byte chunks (8 bf16 each)
// dotted with xin (LDS). A row is one unit of work for a wave (or, when the
// block has fewer rows than waves, an equal part of a row); wave w takes units
// w, w + NW, ... and each lane every 64th chunk of a unit, so a wave reads
// whole 1 KB spans and reduces once per unit. Chunk q*64 + lane of the block's
// unit-major order (q = unit * cpu + i) is the lane's i-th chunk of that unit.
struct GemvPlan {
    int nrows, sf_log2, cpu, units;  // parts per row (log2), chunks per lane per unit, units
    int staged;                      // leading q-spans staged in LDS
};

__device__ __forceinline__ GemvPlan gemv_plan(int nrows, int cpr) {
    GemvPlan g;
    g.nrows = nrows;
    const int cpl = cpr >> 6;
    int lg = 0;
    while ((nrows << lg) < NW && cpl % (2 << lg) == 0) ++lg;
    g.sf_log2 = lg;
    g.cpu = cpl >> lg;
    g.units = nrows << lg;
    const int spans = g.units * g.cpu;
    g.staged = spans < STAGE / 64 ? spans : STAGE / 64;
    return g;
}

// The rows of a GEMV phase: up to three runs of consecutive rows of row-major
// bf16 matrices with `cols` columns, concatenated.
struct RowMap {
    const uint16_t *base[3];
    int rows[3];
    int cols;
};

__device__ __forceinline__ const uint16_t *row_ptr(const RowMap &m, int r) {
    if (r < m.rows[0]) return m.base[0] + (size_t)r * m.cols;
    r -= m.rows[0];
    if (r < m.rows[1]) return m.base[1] + (size_t)r * m.cols;
    r -= m.rows[1];
    return m.base[2] + (size_t)r * m.cols;
}

// The same rows without the first `skip`.
__device__ __forceinline__ RowMap row_skip(RowMap m, int skip) {
    for (int i = 0; i < 3; ++i) {
        const int d = skip < m.rows[i] ? skip : m.rows[i];
        m.base[i] += (size_t)d * m.cols;
        m.rows[i] -= d;
        skip -= d;
    }
    return m;
}

// Column chunk of this lane's chunk in span q.
__device__ __forceinline__ int gemv_col(const GemvPlan &g, int q) {
    const int u = q / g.cpu, i = q - u * g.cpu;
    const int part = u & ((1 << g.sf_log2) - 1);
    return (part * g.cpu + i) * 64 + (threadIdx.x & 63);
}

// Address of this lane's chunk in span q, and its column chunk.
__device__ __forceinline__ const uint4 *gemv_chunk(const GemvPlan &g, const RowMap &m, int q, int &col) {
    const int row = (q / g.cpu) >> g.sf_log2;
    col = gemv_col(g, q);
    return reinterpret_cast<const uint4 *>(row_ptr(m, row)) + col;
}

// Staging waves load the leading spans of the GEMV's weights into LDS; they
// do not depend on the input the block is about to wait for.
__device__ __forceinline__ void gemv_stage(Shared &sh, const GemvPlan &g, const RowMap &m) {
    const int wave = threadIdx.x >> 6;
    for (int q = wave; q < g.staged; q += NW) {
        int col;
        lds_dma16(gemv_chunk(g, m, q, col), sh.stage + q * 64);
    }
}

// Staging waves copy `bytes` (a multiple of 16) from src into LDS at dst.
__device__ __forceinline__ void stage_small(const void *src, void *dst, int bytes) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int chunks = bytes >> 4;
    for (int c0 = wave * 64; c0 < chunks; c0 += NW * 64)
        if (c0 + lane < chunks)
            lds_dma16(reinterpret_cast<const uint4 *>(src) + c0 + lane, reinterpret_cast<uint4 *>(dst) + c0);
}

// Every wave waits for its staging loads, then everyone syncs.
__device__ __forceinline__ void stage_ready() {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
}

__device__ __forceinline__ float dot8(const Shared &sh, const uint4 &w, int col, float acc) {
    const float4 *x4 = reinterpret_cast<const float4 *>(sh.xin) + col * 2;
    const float4 a = x4[0], b = x4[1];
    float wf[8];
    unpack8(w, wf);
    acc = fmaf(wf[0], a.x, acc);
    acc = fmaf(wf[1], a.y, acc);
    acc = fmaf(wf[2], a.z, acc);
    acc = fmaf(wf[3], a.w, acc);
    acc = fmaf(wf[4], b.x, acc);
    acc = fmaf(wf[5], b.y, acc);
    acc = fmaf(wf[6], b.z, acc);
    acc = fmaf(wf[7], b.w, acc);
    return acc;
}

// res[r] = row r . xin for the GEMV whose leading spans gemv_stage staged
// (stage_ready must have run); the rest streams from memory with B chunks per
// lane in flight across unit boundaries.
__device__ __forceinline__ void gemv_run(Shared &sh, const GemvPlan &g, const RowMap &m) {
    constexpr int B = 8;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // This wave's spans: q = (wave + k*NW) * cpu + i, visited in order k, i.
    const int nq = g.units > wave ? ((g.units - wave + NW - 1) / NW) * g.cpu : 0;
    float acc = 0.f;
    int k = 0, i = 0;
    auto span = [&](int kk, int ii) { return (wave + kk * NW) * g.cpu + ii; };
    auto finish = [&]() {
        const float s = wave_sum_dpp(acc);
        if (lane == 0) sh.part[wave + k * NW] = s;
        acc = 0.f;
        i = 0;
        ++k;
    };
    int t = 0;
    for (; t < nq && span(k, i) < g.staged; ++t) {
        const int q = span(k, i);
        acc = dot8(sh, sh.stage[q * 64 + lane], gemv_col(g, q), acc);
        if (++i == g.cpu) finish();
    }
    for (; t < nq; t += B) {
        uint4 w[B];
        int cols[B];
        int kk = k, ii = i;
#pragma unroll
        for (int b = 0; b < B; ++b) {
            if (t + b < nq) w[b] = *gemv_chunk(g, m, span(kk, ii), cols[b]);
            if (++ii == g.cpu) {
                ii = 0;
                ++kk;
            }
        }
#pragma unroll
        for (int b = 0; b < B; ++b) {
            if (t + b < nq) {
                acc = dot8(sh, w[b], cols[b], acc);
                if (++i == g.cpu) finish();
            }
        }
    }
    __syncthreads();
    const int sf = 1 << g.sf_log2;
    for (int r = tid; r < g.nrows; r += NT) {
        float s = 0.f;
        for (int q = 0; q < sf; ++q) s += sh.part[r * sf + q];
        sh.res[r] = s;
    }
    __syncthreads();
}

__device__ __forceinline__ void load_kv8(const void *base, int bf16, long long idx, float f[8]) {
    if (bf16) {
        unpack8(*reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(base) + idx), f);
    } else {
        const float4 *p = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(base) + idx);
        float4 a = p[0], b = p[1];
        f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
        f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    }
}

__device__ __forceinline__ float load_kv1(const void *base, int bf16, long long idx) {
    return bf16 ? bf16_to_f32(reinterpret_cast<const uint16_t *>(base)[idx]) : reinterpret_cast<const float *>(base)[idx];
}

__device__ __forceinline__ void store_kv1(void *base, int bf16, long long idx, float v) {
    if (bf16)
        reinterpret_cast<uint16_t *>(base)[idx] = f32_to_bf16(v);
    else
        reinterpret_cast<float *>(base)[idx] = v;
}

// RMSNorm (optional gain) and RoPE of one head held in LDS, by one wave: lane
// l holds the pairs (l + 64k, l + 64k + hd/2).
__device__ __forceinline__ void norm_rope_head(float *h, int hd, const uint16_t *gain, float eps, const float *ang) {
    const int lane = threadIdx.x & 63, half = hd / 2;
    float a[2], b[2];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = lane + 64 * k;
        a[k] = i < half ? h[i] : 0.f;
        b[k] = i < half ? h[i + half] : 0.f;
        ss += a[k] * a[k] + b[k] * b[k];
    }
    if (gain) {
        ss = wave_sum(ss);
        const float scale = 1.0f / sqrtf(ss / (float)hd + eps);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int i = lane + 64 * k;
            if (i < half) {
                a[k] = a[k] * (scale * bf16_to_f32(gain[i]));
                b[k] = b[k] * (scale * bf16_to_f32(gain[i + half]));
            }
        }
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = lane + 64 * k;
        if (i < half) {
            const float c = ang[2 * i], s = ang[2 * i + 1];
            h[i] = a[k] * c - b[k] * s;
            h[i + half] = b[k] * c + a[k] * s;
        }
    }
}

// One attention item: KV head g, positions [s0, s1) of the token at `pos`.
// Leaves the unnormalized accumulator in sh.part ([gg][hd]) and (m, l) in sh.st_m/st_l.
template <int HD, int G>
__device__ __forceinline__ void attend(Shared &sh, const DecodeParams &p, const void *kc, const void *vc, long long pos,
                       long long s0, long long s1, int npre) {
    constexpr int LPK = HD / 8, KPW = 64 / LPK, KPB = NW * KPW, NP = NT / HD;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, sub = lane % LPK;
    const float scale = 1.0f / sqrtf((float)HD);
    const float *hq = sh.hqkv, *hk = sh.hqkv + G * HD, *hv = sh.hqkv + (G + 1) * HD;
    // Positions s0 .. s0+npre-1 are staged in LDS: npre K rows, then npre V rows.
    const char *kl = reinterpret_cast<const char *>(sh.stage);
    const size_t row_bytes = (size_t)HD * (p.kv_bf16 ? 2 : 4);
    const char *vl = kl + npre * row_bytes;
    float qf[G][8];
#pragma unroll
    for (int gg = 0; gg < G; ++gg)
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[gg][i] = hq[gg * HD + sub * 8 + i];
    if (tid < MAXG) {
        sh.st_m[tid] = -INFINITY;
        sh.st_l[tid] = 0.f;
    }
    const int d = tid % HD, pt = tid / HD;
    float acc[G];
#pragma unroll
    for (int gg = 0; gg < G; ++gg) acc[gg] = 0.f;
    for (long long c0 = s0; c0 < s1; c0 += SUB) {
        const int cnt = (int)(s1 - c0 < SUB ? s1 - c0 : SUB);
        for (int j0 = 0; j0 < cnt; j0 += KPB) {
            const int j = j0 + wave * KPW + lane / LPK;
            const long long jp = c0 + j;
            float kf[8];
            if (j < cnt && jp - s0 < npre) {
                load_kv8(kl + (jp - s0) * row_bytes, p.kv_bf16, sub * 8, kf);
            } else if (j < cnt && jp < pos) {
                load_kv8(kc, p.kv_bf16, jp * HD + sub * 8, kf);
            } else if (j < cnt) {
#pragma unroll
                for (int i = 0; i < 8; ++i) kf[i] = hk[sub * 8 + i];
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) kf[i] = 0.f;
            }
#pragma unroll
            for (int gg = 0; gg < G; ++gg) {
                float s = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) s = fmaf(qf[gg][i], kf[i], s);
                s = group_sum<LPK>(s);
                if (j < cnt && sub == 0) sh.scores[gg][j] = scale * s;
            }
        }
        __syncthreads();
        for (int gg = wave; gg < G; gg += NW) {
            float m = -INFINITY;
            for (int j = lane; j < cnt; j += 64) m = fmaxf(m, sh.scores[gg][j]);
            m = wave_max(m);
            const float m_old = sh.st_m[gg], m_new = fmaxf(m_old, m);
            float l = 0.f;
            for (int j = lane; j < cnt; j += 64) {
                const float e = expf(sh.scores[gg][j] - m_new);
                sh.scores[gg][j] = e;
                l += e;
            }
            l = wave_sum(l);
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
        for (int j = pt; j < cnt; j += NP) {
            const long long jp = c0 + j;
            const float v = jp - s0 < npre ? load_kv1(vl + (jp - s0) * row_bytes, p.kv_bf16, d)
                            : jp < pos     ? load_kv1(vc, p.kv_bf16, jp * HD + d)
                                           : hv[d];
#pragma unroll
            for (int gg = 0; gg < G; ++gg) acc[gg] = fmaf(sh.scores[gg][j], v, acc[gg]);
        }
        __syncthreads();
    }
    // Sum the NP position groups: part[gg][d].
    for (int q = 0; q < NP; ++q) {
        if (pt == q) {
#pragma unroll
            for (int gg = 0; gg < G; ++gg) sh.part[gg * HD + d] = (q == 0 ? 0.f : sh.part[gg * HD + d]) + acc[gg];
        }
        __syncthreads();
    }
}

template <int HD, int G>
__device__ __forceinline__ bool attention_phase(Shared &sh, const DecodeParams &p, int layer, long long pos, unsigned eA,
                                unsigned eB) {
    const int tid = threadIdx.x, wave = tid >> 6;
    const int nkv = p.n_kv_heads;
    const int qd = p.n_heads * HD;
    const LayerWeights &W = p.layers[layer];
    const size_t per = (size_t)nkv * p.max_len * HD;  // elements per (layer, k|v)
    const int n_items = nkv * p.n_splits;
    const int n_act = (int)(pos / p.chunk) + 1;  // splits holding positions 0..pos
    for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
        const int g = item % nkv, sp = item / nkv;
        const long long s0 = (long long)sp * p.chunk;
        if (s0 > pos) continue;
        const long long s1 = s0 + p.chunk < pos + 1 ? s0 + p.chunk : pos + 1;
        const size_t elem = p.kv_bf16 ? 2 : 4;
        char *kvbase = static_cast<char *>(p.kv);
        void *kc = kvbase + ((size_t)(layer * 2 + 0) * per + (size_t)g * p.max_len * HD) * elem;
        void *vc = kvbase + ((size_t)(layer * 2 + 1) * per + (size_t)g * p.max_len * HD) * elem;
        // Cached rows before pos do not depend on this step: the staging waves
        // load the first of them into LDS while the q/k/v rows are computed.
        const int row_chunks = (int)(HD * elem / 16);
        const long long cached = (s1 < pos ? s1 : pos) - s0;
        const int cap = STAGE / (2 * row_chunks);
        const int npre = (int)(cached < cap ? (cached > 0 ? cached : 0) : cap);
        const int kv_spans = (npre * row_chunks * 2 + 63) / 64;
        __syncthreads();  // the stage may still be read by the previous item
        {
            for (int q = wave; q < kv_spans; q += NW) {
                const int idx = q * 64 + (tid & 63);
                if (idx < npre * row_chunks * 2) {
                    const int half = idx / (npre * row_chunks), rem = idx - half * npre * row_chunks;
                    const int prow = rem / row_chunks, c = rem - prow * row_chunks;
                    const char *src = static_cast<const char *>(half ? vc : kc) + (size_t)(s0 + prow) * HD * elem;
                    lds_dma16(reinterpret_cast<const uint4 *>(src) + c, sh.stage + q * 64);
                }
            }
        }
        if (W.q_norm) stage_small(W.q_norm, sh.qk_gain, HD * 2);
        if (W.k_norm) stage_small(W.k_norm, sh.qk_gain + HD, HD * 2);
        stage_small(p.rope + pos * HD, sh.rope_row, HD * 4);
        // This head group's raw q heads, k and v, contiguous in the exchange.
        if (!wait_vec(p, p.xchg_qkv + (size_t)g * (G + 2) * HD, (G + 2) * HD, eA, sh.hqkv)) return false;
        stage_ready();
        float *hk = sh.hqkv + G * HD, *hv = sh.hqkv + (G + 1) * HD;
        for (int h = wave; h <= G; h += NW) {
            const uint16_t *gain = h < G ? (W.q_norm ? sh.qk_gain : nullptr) : (W.k_norm ? sh.qk_gain + HD : nullptr);
            norm_rope_head(sh.hqkv + h * HD, HD, gain, p.eps, sh.rope_row);
        }
        __syncthreads();
        if (pos >= s0 && pos < s0 + p.chunk) {
            for (int i = tid; i < HD; i += NT) {
                store_kv1(kc, p.kv_bf16, pos * HD + i, hk[i]);
                store_kv1(vc, p.kv_bf16, pos * HD + i, hv[i]);
            }
        }
        attend<HD, G>(sh, p, kc, vc, pos, s0, s1, npre);
        if (n_act == 1) {
            if (wave == PUB)
                for (int i = tid & 63; i < G * HD; i += 64) {
                    const int gg = i / HD;
                    publish(p.xchg_att, qd, g * G * HD + i, sh.part[i] / sh.st_l[gg], eB, kReplicas);
                }
            continue;
        }
        // Several splits: store this one's partial, then the last to arrive merges.
        float *pp = p.att_part;
        const int stride = HD + 2;
        for (int i = tid; i < G * HD; i += NT) {
            const int gg = i / HD, dd = i % HD;
            float *slot = pp + ((size_t)(g * G + gg) * p.n_splits + sp) * stride;
            __hip_atomic_store(reinterpret_cast<unsigned *>(slot + dd), __float_as_uint(sh.part[i]), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            if (dd == 0) {
                __hip_atomic_store(reinterpret_cast<unsigned *>(slot + HD), __float_as_uint(sh.st_m[gg]),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(reinterpret_cast<unsigned *>(slot + HD + 1), __float_as_uint(sh.st_l[gg]),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        __builtin_amdgcn_s_waitcnt(0);  // the partial's stores are complete before the count
        __syncthreads();
        if (tid == 0) {
            unsigned *cnt = p.att_count + (size_t)layer * nkv + g;
            const unsigned prev = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int last = prev == (unsigned)(n_act - 1);
            if (last) {
                // Reset for the next step, complete before this merge is published.
                __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __builtin_amdgcn_s_waitcnt(0);
            }
            sh.flag = last;
        }
        __syncthreads();
        if (!sh.flag) continue;
        for (int i = tid; i < G * HD; i += NT) {
            const int gg = i / HD, dd = i % HD;
            const float *base = pp + (size_t)(g * G + gg) * p.n_splits * stride;
            float m = -INFINITY;
            for (int s = 0; s < n_act; ++s)
                m = fmaxf(m, __uint_as_float(__hip_atomic_load(reinterpret_cast<const unsigned *>(base + s * stride + HD),
                                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)));
            float l = 0.f, a = 0.f;
            for (int s = 0; s < n_act; ++s) {
                const float ms = __uint_as_float(__hip_atomic_load(
                    reinterpret_cast<const unsigned *>(base + s * stride + HD), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
                const float ls = __uint_as_float(__hip_atomic_load(
                    reinterpret_cast<const unsigned *>(base + s * stride + HD + 1), __ATOMIC_RELAXED,
                    __HIP_MEMORY_SCOPE_AGENT));
                const float as = __uint_as_float(__hip_atomic_load(
                    reinterpret_cast<const unsigned *>(base + s * stride + dd), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
                if (ms != -INFINITY) {
                    const float sc = expf(ms - m);
                    l += ls * sc;
                    a += as * sc;
                }
            }
            publish(p.xchg_att, qd, g * G * HD + i, a / l, eB, kReplicas);
        }
    }
    return true;
}

// Block 0 notes ticks in LDS (a global store here would add its acknowledgement
// to the next wait of the noting wave) and writes a traced step out at its end.
__device__ __forceinline__ void trace_at(Shared &sh, const DecodeParams &p, int s, int slot, int which) {
    if (p.trace && blockIdx.x == 0 && threadIdx.x == PUB * 64 && s < p.trace_steps && slot < TRACE_SLOTS)
        sh.ticks[slot * TRACE_POINTS + which] = (unsigned)__builtin_amdgcn_s_memrealtime();
}

__device__ __forceinline__ void trace_flush(Shared &sh, const DecodeParams &p, int s) {
    if (!p.trace || blockIdx.x != 0 || s >= p.trace_steps) return;
    __syncthreads();
    const int words = (p.n_layers * 5 + 2) * TRACE_POINTS;
    for (int i = threadIdx.x; i < words; i += NT)
        p.trace[1 + (size_t)s * words + i] = i < TRACE_SLOTS * TRACE_POINTS ? sh.ticks[i] : 0;
    __syncthreads();
    if (threadIdx.x == 0) for (int i = 0; i < TRACE_SLOTS * TRACE_POINTS; ++i) sh.ticks[i] = 0;
}

template <int HD, int G>
__global__ __launch_bounds__(NT) void decode_kernel(DecodeParams p) {
    __shared__ Shared sh;
    const int tid = threadIdx.x, blk = blockIdx.x, nblk = gridDim.x;
    const int rep = blk % kReplicas;
    const int H = p.hidden, I = p.intermediate, L = p.n_layers, V = p.vocab;
    const int qd = p.n_heads * HD, kvd = p.n_kv_heads * HD, Rqkv = qd + 2 * kvd;
    // This block's rows of each phase.
    const int o0 = (int)((long long)blk * H / nblk), o1 = (int)((long long)(blk + 1) * H / nblk), n_own = o1 - o0;
    const int q0 = (int)((long long)blk * Rqkv / nblk), q1 = (int)((long long)(blk + 1) * Rqkv / nblk);
    const int j0 = (int)((long long)blk * I / nblk), j1 = (int)((long long)(blk + 1) * I / nblk), nj = j1 - j0;
    const int v0 = (int)((long long)blk * V / nblk), v1 = (int)((long long)(blk + 1) * V / nblk);
    const int PH = 5 * L + 2;  // phases per step: 5 per layer, output projection, pick
    // The q/k/v rows [q0, q1) of the block, as runs of the three matrices.
    const int qa = q0 < qd ? q0 : qd, qb = q1 < qd ? q1 : qd;
    const int ka = q0 < qd ? qd : (q0 < qd + kvd ? q0 : qd + kvd), kb = q1 < qd + kvd ? (q1 > qd ? q1 : qd) : qd + kvd;
    const int va = q0 > qd + kvd ? q0 : qd + kvd, vb = q1 > qd + kvd ? q1 : qd + kvd;

    StepState *st = p.step;
    const long long pos0 = st->pos, step0 = st->step;
    unsigned token = st->token;
    float *const keep = st->logits_out;
    if (p.trace && blk == 0 && tid == 0) {
        p.trace[0] = __builtin_amdgcn_s_memrealtime() & 0xffffffffull;
        for (int i = 0; i < TRACE_SLOTS * TRACE_POINTS; ++i) sh.ticks[i] = 0;
    }

    for (int s = 0; s < p.steps; ++s) {
        const long long pos = pos0 + s;
        const unsigned eb = p.epoch_base + (unsigned)s * (unsigned)PH;
        uint64_t best = 0;
        for (int ph = 0; ph < PH; ++ph) {
            const int l = ph < 5 * L ? ph / 5 : L - 1;
            const int kind = ph < 5 * L ? ph % 5 : (ph == 5 * L ? 5 : 6);
            const unsigned e = eb + (unsigned)ph + 1;  // the epoch this phase publishes; its input carries e - 1
            const LayerWeights &W = p.layers[l];
            if (kind == 1) {
                // ---- B: attention (blocks holding an attention item)
                trace_at(sh, p, s, ph, 0);
                if (!attention_phase<HD, G>(sh, p, l, pos, e - 1, e)) return;
                trace_at(sh, p, s, ph, 3);
                continue;
            }
            if (kind == 6) {
                // ---- G: the greedy pick, reduced by every block for itself
                if (!wait_vec(p, p.xchg_am + (size_t)rep * 2 * nblk, 2 * nblk, e - 1, sh.xin)) return;
                trace_at(sh, p, s, ph, 0);
                uint64_t b = 0;
                for (int i = tid; i < nblk; i += NT)
                    b = max_u64(b, ((uint64_t)__float_as_uint(sh.xin[2 * i]) << 32) | __float_as_uint(sh.xin[2 * i + 1]));
                b = wave_max_u64(b);
                __syncthreads();
                if ((tid & 63) == 0) sh.red64[tid >> 6] = b;
                __syncthreads();
                b = 0;
                for (int w = 0; w < NW; ++w) b = max_u64(b, sh.red64[w]);
                token = argmax_index(b);
                if (blk == 0 && tid == 0 && st->tokens_out) st->tokens_out[step0 + s + 1] = token;
                trace_at(sh, p, s, ph, 3);
                trace_flush(sh, p, s);
                continue;
            }
            // ---- A GEMV phase: A (attention norm + q/k/v), C (o + residual),
            // D (MLP norm + gate/up + SiLU), E (down + residual), F (final norm +
            // output projection + argmax).
            RowMap m;
            m.rows[1] = m.rows[2] = 0;
            m.base[1] = m.base[2] = nullptr;
            const uint16_t *gain = nullptr;
            const u64 *in = nullptr;
            int in_n = 0, nrows = 0;
            if (kind == 0) {
                m.base[0] = W.q + (size_t)qa * H;
                m.rows[0] = qb - qa;
                m.base[1] = W.k + (size_t)(ka - qd) * H;
                m.rows[1] = kb - ka;
                m.base[2] = W.v + (size_t)(va - qd - kvd) * H;
                m.rows[2] = vb - va;
                m.cols = H;
                nrows = q1 - q0;
                gain = W.attn_norm;
                if (l > 0) in = p.xchg_x + (size_t)rep * H, in_n = H;
            } else if (kind == 2) {
                m.base[0] = W.o + (size_t)o0 * qd;
                m.rows[0] = n_own;
                m.cols = qd;
                nrows = n_own;
                in = p.xchg_att + (size_t)rep * qd, in_n = qd;
            } else if (kind == 3) {
                m.base[0] = W.gate + (size_t)j0 * H;
                m.rows[0] = nj;
                m.base[1] = W.up + (size_t)j0 * H;
                m.rows[1] = nj;
                m.cols = H;
                nrows = 2 * nj;
                gain = W.mlp_norm;
                in = p.xchg_x + (size_t)rep * H, in_n = H;
            } else if (kind == 4) {
                m.base[0] = W.down + (size_t)o0 * I;
                m.rows[0] = n_own;
                m.cols = I;
                nrows = n_own;
                in = p.xchg_h + (size_t)rep * I, in_n = I;
            } else {
                m.base[0] = p.lm_head + (size_t)v0 * H;
                m.rows[0] = v1 - v0;
                m.cols = H;
                nrows = v1 - v0;
                gain = p.norm;
                in = p.xchg_x + (size_t)rep * H, in_n = H;
            }
            for (int r0 = 0; r0 < nrows; r0 += MAX_RES) {
                const int nr = nrows - r0 < MAX_RES ? nrows - r0 : MAX_RES;
                const RowMap mp = row_skip(m, r0);
                const GemvPlan g = gemv_plan(nr, m.cols / 8);
                gemv_stage(sh, g, mp);
                if (r0 == 0) {
                    if (gain) stage_small(gain, sh.gain, H * 2);
                    if (in) {
                        if (!wait_vec(p, in, in_n, e - 1, sh.xin)) return;
                    } else {
                        // The first layer's input: the token's embedding row.
                        __syncthreads();
                        const uint4 *row = reinterpret_cast<const uint4 *>(p.embed + (size_t)token * H);
                        for (int c = tid; c < H / 8; c += NT) {
                            float f[8];
                            unpack8(row[c], f);
#pragma unroll
                            for (int e8 = 0; e8 < 8; ++e8) sh.xin[c * 8 + e8] = f[e8];
                        }
                        __syncthreads();
                        for (int i = tid; i < n_own; i += NT) sh.xown[i] = sh.xin[o0 + i];
                    }
                    trace_at(sh, p, s, ph, 0);
                }
                stage_ready();
                if (r0 == 0) {
                    trace_at(sh, p, s, ph, 1);
                    if (gain) rmsnorm_lds(sh, H, p.eps);
                }
                gemv_run(sh, g, mp);
                if (r0 == 0) trace_at(sh, p, s, ph, 2);
                if (kind == 5) {
                    for (int t = tid; t < nr; t += NT) {
                        const int row = v0 + r0 + t;
                        const float lg = sh.res[t];
                        p.logits[row] = lg;
                        if (keep) keep[(size_t)(step0 + s) * V + row] = lg;
                        best = max_u64(best, argmax_pack(lg, (uint32_t)row));
                    }
                    continue;
                }
                // Publishing is the last wave's job (it never polls).
                for (int t = tid - PUB * 64; t >= 0 && t < nr; t += 64) {
                    if (kind == 0) {
                        // Exchange layout per KV group g: its G q heads, its k head, its v head.
                        const int r = q0 + t;
                        int slot;
                        if (r < qd) {
                            const int h = r / HD, gq = h / G;
                            slot = gq * (G + 2) * HD + (h - gq * G) * HD + (r - h * HD);
                        } else if (r < qd + kvd) {
                            const int gk = (r - qd) / HD;
                            slot = gk * (G + 2) * HD + G * HD + (r - qd - gk * HD);
                        } else {
                            const int gv = (r - qd - kvd) / HD;
                            slot = gv * (G + 2) * HD + (G + 1) * HD + (r - qd - kvd - gv * HD);
                        }
                        publish(p.xchg_qkv, Rqkv, slot, sh.res[t], e, 1);
                    } else if (kind == 3) {
                        if (t < nj) publish(p.xchg_h, I, j0 + t, silu(sh.res[t]) * sh.res[nj + t], e, kReplicas);
                    } else {
                        sh.xown[t] += sh.res[t];
                        publish(p.xchg_x, H, o0 + t, sh.xown[t], e, kReplicas);
                    }
                }
            }
            if (kind == 5) {
                // This block's argmax, as (key, inverted index) words.
                best = wave_max_u64(best);
                if ((tid & 63) == 0) sh.red64[tid >> 6] = best;
                __syncthreads();
                if (tid == PUB * 64) {
                    uint64_t b = 0;
                    for (int w = 0; w < NW; ++w) b = max_u64(b, sh.red64[w]);
                    for (int r = 0; r < kReplicas; ++r) {
                        u64 *am = p.xchg_am + (size_t)r * 2 * nblk;
                        __hip_atomic_store(am + 2 * blk, ((u64)e << 32) | (b >> 32), __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                        __hip_atomic_store(am + 2 * blk + 1, ((u64)e << 32) | (b & 0xffffffffull), __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
            }
            trace_at(sh, p, s, ph, 3);
        }
    }
    if (blk == 0 && tid == 0) {
        st->pos = pos0 + p.steps;
        st->step = step0 + p.steps;
        st->token = token;
    }
}

}  // namespace

bool decode_supported(int hidden, int intermediate, int n_heads, int n_kv_heads, int head_dim, int vocab,
                      int blocks) {
    if (head_dim != 128 || blocks <= 0) return false;
    const int g = n_kv_heads > 0 && n_heads % n_kv_heads == 0 ? n_heads / n_kv_heads : 0;
    if (g != 1 && g != 2 && g != 4 && g != 8) return false;
    // Every row must span whole waves of 16-byte chunks, and fit the LDS input.
    const int cols[3] = {hidden, n_heads * head_dim, intermediate};
    for (int c : cols)
        if (c % 512 != 0 || c > MAX_COLS) return false;
    // Rows per block in each phase must fit the LDS partials.
    auto per = [&](long long n) { return (int)((n + blocks - 1) / blocks); };
    const int rqkv = (n_heads + 2 * n_kv_heads) * head_dim;
    if (per(hidden) > MAX_OWN || hidden > MAX_H) return false;
    if (per(rqkv) > MAX_RES || 2 * per(intermediate) > MAX_RES) return false;
    if (2 * blocks > MAX_COLS || vocab <= 0) return false;
    return true;
}

int decode_blocks(int device) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return 0;
    return prop.multiProcessorCount;
}

hipError_t launch_decode(hipStream_t s, const DecodeParams &p, int blocks) {
    DecodeParams copy = p;
    void *args[] = {&copy};
    const void *fn = nullptr;
    switch (p.n_heads / p.n_kv_heads) {
    case 1: fn = (const void *)decode_kernel<128, 1>; break;
    case 2: fn = (const void *)decode_kernel<128, 2>; break;
    case 4: fn = (const void *)decode_kernel<128, 4>; break;
    case 8: fn = (const void *)decode_kernel<128, 8>; break;
    default: return hipErrorInvalidValue;
    }
    return hipLaunchCooperativeKernel(fn, dim3(blocks), dim3(NT), args, 0, s);
}

}  // namespace th
