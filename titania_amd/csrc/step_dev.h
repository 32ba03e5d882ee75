// Device code of the decode-step kernels: the GEMV input builder, row tables,
// and the register-resident attention of one KV head over the whole context.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "device_util.h"
#include "fused.h"
#include "step.h"

namespace th {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

// Builds the block's f32 input in LDS: x = a (+ b), optionally RMSNorm'd with
// gain g (model/cpu.rs:85-94); block 0 keeps the un-normalized sum in x_out.
// Every thread issues all its loads (NV float4 of a, of b
// and 4-element groups of g) before using any, so the input costs one memory
// round trip rather than one per loop iteration.
template <bool NORM, int NV>
__device__ __forceinline__ void build_input(float *xs, const float *a, const float *b, int n, const uint16_t *g,
                                            float eps, float *x_out, float *red) {
    const int tid = threadIdx.x;
    const int n4 = n >> 2;
    const float4 *a4 = reinterpret_cast<const float4 *>(a);
    const float4 *b4 = reinterpret_cast<const float4 *>(b);
    const uint2 *g4 = reinterpret_cast<const uint2 *>(g);
    float4 va[NV], vb[NV];
    uint2 vg[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int i = tid + k * kThreads;
        if (i < n4) {
            va[k] = a4[i];
            if (b) vb[k] = b4[i];
            if (NORM) vg[k] = g4[i];
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int i = tid + k * kThreads;
        if (i < n4) {
            float4 v = va[k];
            if (b) {
                v.x = v.x + vb[k].x;
                v.y = v.y + vb[k].y;
                v.z = v.z + vb[k].z;
                v.w = v.w + vb[k].w;
            }
            va[k] = v;
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            if (!NORM) reinterpret_cast<float4 *>(xs)[i] = v;
        }
    }
    if (x_out && blockIdx.x == 0) {  // every block holds the sum; the first keeps it
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int i = tid + k * kThreads;
            if (i < n4) reinterpret_cast<float4 *>(x_out)[i] = va[k];
        }
    }
    if (!NORM) {
        __syncthreads();
        return;
    }
    ss = wave_sum_dpp(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    float total = 0.f;
    for (int w = 0; w < kWaves; ++w) total += red[w];
    const float scale = 1.0f / sqrtf(total / (float)n + eps);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int i = tid + k * kThreads;
        if (i < n4) {
            float4 v = va[k];
            v.x = v.x * (scale * bf16_lo(vg[k].x));
            v.y = v.y * (scale * bf16_hi(vg[k].x));
            v.z = v.z * (scale * bf16_lo(vg[k].y));
            v.w = v.w * (scale * bf16_hi(vg[k].y));
            reinterpret_cast<float4 *>(xs)[i] = v;
        }
    }
    __syncthreads();
}

__device__ __forceinline__ float dot8(const float *xs, const uint4 &w, int col, float acc) {
    const float4 *x4 = reinterpret_cast<const float4 *>(xs) + col * 2;
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

// Rows of a GEMV: up to three runs of consecutive rows of row-major matrices
// with `cols` columns, concatenated.
struct Rows {
    const uint16_t *base[3];
    int count[3];
};

__device__ __forceinline__ const uint4 *row_at(const Rows &m, int r, int cols) {
    const uint16_t *p;
    if (r < m.count[0]) p = m.base[0] + (size_t)r * cols;
    else if (r < m.count[0] + m.count[1]) p = m.base[1] + (size_t)(r - m.count[0]) * cols;
    else p = m.base[2] + (size_t)(r - m.count[0] - m.count[1]) * cols;
    return reinterpret_cast<const uint4 *>(p);
}

__device__ __forceinline__ void lds_row8(const float *row, int sub, float f[8]) {
    const float4 a = reinterpret_cast<const float4 *>(row)[sub * 2], b = reinterpret_cast<const float4 *>(row)[sub * 2 + 1];
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}
__device__ __forceinline__ void lds_row8(const uint16_t *row, int sub, float f[8]) {
    unpack8(reinterpret_cast<const uint4 *>(row)[sub], f);
}
// Cached K/V rows held in registers: in the score pass a lane holds dims
// [8*sub, 8*sub + 8) of its keys, in the value pass dims [4*d4, 4*d4 + 4).
template <typename KV> struct KvRegs;
template <> struct KvRegs<float> {
    struct K { float4 a, b; };
    using V = float4;
    static constexpr int kRows = 64;  // positions per pass
    __device__ static K load_k(const float *row, int sub) {
        const float4 *p = reinterpret_cast<const float4 *>(row) + sub * 2;
        return K{p[0], p[1]};
    }
    __device__ static void unpack_k(const K &k, float f[8]) {
        f[0] = k.a.x; f[1] = k.a.y; f[2] = k.a.z; f[3] = k.a.w;
        f[4] = k.b.x; f[5] = k.b.y; f[6] = k.b.z; f[7] = k.b.w;
    }
    __device__ static V load_v(const float *row, int d4) { return reinterpret_cast<const float4 *>(row)[d4]; }
    __device__ static void unpack_v(const V &v, float f[4]) {
        f[0] = v.x; f[1] = v.y; f[2] = v.z; f[3] = v.w;
    }
};
template <> struct KvRegs<uint16_t> {
    using K = uint4;
    using V = uint2;
    static constexpr int kRows = 128;
    __device__ static K load_k(const uint16_t *row, int sub) { return reinterpret_cast<const uint4 *>(row)[sub]; }
    __device__ static void unpack_k(const K &k, float f[8]) { unpack8(k, f); }
    __device__ static V load_v(const uint16_t *row, int d4) { return reinterpret_cast<const uint2 *>(row)[d4]; }
    __device__ static void unpack_v(const V &v, float f[4]) {
        f[0] = bf16_lo(v.x); f[1] = bf16_hi(v.x);
        f[2] = bf16_lo(v.y); f[3] = bf16_hi(v.y);
    }
};

// The end of a chunked launch for dimension d of q head h, given this chunk's
// (sum, max, denominator): with one chunk holding positions, the output;
// else chunks 1.. publish theirs as epoch words at
// xw + (h * n_chunks + split) * (128 + 2) and chunk 0 polls them (eight
// chunks at a time) and merges all in chunk order into a.out.
__device__ __forceinline__ void chunk_finish(const StepAttnArgs &a, long long h, int d, float sm, float sm_m,
                                             float sm_l, unsigned long long *xw, int n_chunks, int split,
                                             int n_live, unsigned epoch, unsigned *err) {
    constexpr int HD = 128;
    if (n_live == 1) {
        a.out[h * HD + d] = sm / sm_l;
        return;
    }
    unsigned long long *hw = xw + (size_t)h * n_chunks * (HD + 2);
    auto tag = [&](float v) { return ((unsigned long long)epoch << 32) | __float_as_uint(v); };
    if (split > 0) {
        unsigned long long *cw = hw + (size_t)split * (HD + 2);
        __hip_atomic_store(cw + d, tag(sm), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (d == 0) {
            __hip_atomic_store(cw + HD, tag(sm_m), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(cw + HD + 1, tag(sm_l), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }
    constexpr int PG = 8;
    float num = sm, m = sm_m, den = sm_l;
    for (int c0 = 1; c0 < n_live; c0 += PG) {
        unsigned long long wa[PG], wm[PG], wl[PG];
        for (int it = 0;; ++it) {
            bool ok = true;
#pragma unroll
            for (int i = 0; i < PG; ++i) {
                if (c0 + i >= n_live) break;
                const unsigned long long *cw = hw + (size_t)(c0 + i) * (HD + 2);
                wa[i] = __hip_atomic_load(cw + d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                wm[i] = __hip_atomic_load(cw + HD, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                wl[i] = __hip_atomic_load(cw + HD + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
#pragma unroll
            for (int i = 0; i < PG; ++i) {
                if (c0 + i >= n_live) break;
                ok = ok && (unsigned)(wa[i] >> 32) == epoch && (unsigned)(wm[i] >> 32) == epoch &&
                     (unsigned)(wl[i] >> 32) == epoch;
            }
            if (ok) break;
            if (it >= (1 << 21)) {
                if (d == 0) atomicAdd(err, 1u);
                break;
            }
        }
#pragma unroll
        for (int i = 0; i < PG; ++i) {
            if (c0 + i >= n_live) break;
            const float mc = __uint_as_float((unsigned)wm[i]), mx = fmaxf(m, mc);
            const float s_old = expf(m - mx), s_new = expf(mc - mx);
            num = num * s_old + __uint_as_float((unsigned)wa[i]) * s_new;
            den = den * s_old + __uint_as_float((unsigned)wl[i]) * s_new;
            m = mx;
        }
    }
    a.out[h * HD + d] = num / den;
}

// Attention of one KV head by one block over the positions [s0, s0 + chunk)
// of the context, s0 = split * chunk: the whole context (split 0, chunk
// max_len) or one split of it. The raw q/k/v come from a.qkv, or (WORDS) from
// (value | epoch << 32) words that other blocks of the same launch write,
// polled until they all carry `epoch` (bounded: about 2 s, then *err counts
// the failure and the block goes on). The first pass's cached rows are
// requested before anything else, without waiting for the position: rows past
// the context are read and then ignored (a pass starts below max_len and the
// caches' allocation extends kStepKvTailRows rows past the last head). Later
// passes request their rows as soon as the previous pass has used the
// registers. Reductions are DPP. The output goes to a.out with one split,
// else (sum, max, denominator) partials for launch_attn_combine.
//
// The block's G q heads are qh0 .. qh0 + G - 1 of KV head g (qh0 = g G unless
// a KV head's group is spread over several blocks, of which only the one with
// `append` writes the new key and value).
//
// With `xw` (chunked launches, G = 1): the block covers one chunk of the
// context; chunks past the context return at once. When several chunks hold
// positions, each but the first publishes its (sum, max, denominator) as
// epoch words at xw + (qh0 * n_chunks + split) * (head_dim + 2), and the
// first polls them and merges all, in chunk order, into a.out.
template <int G, typename KV, bool WORDS>
__device__ __forceinline__ void attend_regs(const StepAttnArgs &a, int g, int qh0, bool append, int split,
                                            long long chunk, const unsigned long long *words, unsigned epoch,
                                            unsigned *err, unsigned long long *xw = nullptr, int n_chunks = 1) {
    using R = KvRegs<KV>;
    constexpr int HD = 128, HALF = HD / 2, ROWS = R::kRows;
    constexpr int NK = ROWS / 16;  // keys per lane in the score pass
    constexpr int NV = ROWS / 8;   // keys per lane in the value pass
    constexpr int HPW = (G + 1 + kWaves - 1) / kWaves;
    static_assert(G <= kWaves, "one wave per q head in the softmax");
    static_assert(ROWS <= kStepKvTailRows, "pass longer than the caches' tail");
    __shared__ float hq[G * HD], hk[HD], hv[HD];
    __shared__ float scores[G][ROWS];
    __shared__ float st_m[G], st_l[G], st_a[G];
    __shared__ float red[G][kWaves][HD];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sub = lane & 15, kq = wave * 4 + (lane >> 4);  // score pass: dims 8*sub.., key kq of 16
    const int d4 = tid & 31, pv = tid >> 5;                   // value pass: dims 4*d4.., key pv of 8
    const int qd = a.n_heads * HD, kvd = a.n_kv_heads * HD;
    const long long max_len = a.head_stride / HD;
    const long long s0 = (long long)split * chunk;
    const KV *kc = reinterpret_cast<const KV *>(a.k_cache) + (size_t)g * a.head_stride;
    const KV *vc = reinterpret_cast<const KV *>(a.v_cache) + (size_t)g * a.head_stride;
    typename R::K kr[NK];
    typename R::V vr[NV];
    auto load_k = [&](long long c0) {
#pragma unroll
        for (int i = 0; i < NK; ++i) kr[i] = R::load_k(kc + (c0 + i * 16) * HD + kq * HD, sub);
    };
    auto load_v = [&](long long c0) {
#pragma unroll
        for (int i = 0; i < NV; ++i) vr[i] = R::load_v(vc + (c0 + i * 8) * HD + pv * HD, d4);
    };
    // The position through the scalar cache (the kernel only reads it): a
    // chunk past the context leaves before requesting any rows, and the small
    // loads that depend on the position need no vector wait first.
    const long long pos = *(const __attribute__((address_space(4))) long long *)a.pos;
    const long long len = pos + 1;
    if (xw && s0 >= len) return;  // a chunk past the context (uniform over the block)
    // A range starting past max_len (it has no positions) reads the last rows
    // again, within the caches' tail: the loads need no branch.
    const long long k0 = s0 < max_len ? s0 : max_len - 1;
    if (WORDS) {
        // The q/k/v words come long after the rows: request the rows first.
        load_k(k0);
        load_v(k0);
    }
    const float2 cs = reinterpret_cast<const float2 *>(a.rope + pos * HD)[lane];
    // RMSNorm gains of this wave's heads (q heads 0..G-1, then k), and, from
    // a.qkv, the raw rows: loaded with no branch (rows clamped to valid ones)
    // and used only once the cached rows are requested, so that no wait for
    // them comes before that.
    uint32_t gra[HPW], grb[HPW];
    float ar[HPW], br[HPW], vraw = 0.f;
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
        const int h = min(wave + hh * kWaves, G);
        const uint16_t *gain = h < G ? a.q_norm : a.k_norm;
        const uint16_t *gp = gain ? gain : reinterpret_cast<const uint16_t *>(a.rope);
        gra[hh] = gp[lane];
        grb[hh] = gp[lane + HALF];
        ar[hh] = br[hh] = 0.f;
        if (!WORDS) {
            const float *x = h < G ? a.qkv + (size_t)(qh0 + h) * HD : a.qkv + qd + (size_t)g * HD;
            ar[hh] = x[lane];
            br[hh] = x[lane + HALF];
        }
    }
    if (!WORDS) {
        vraw = a.qkv[qd + kvd + (size_t)g * HD + (tid & (HD - 1))];
        // Here q/k/v are already in memory: the small loads go first, so that
        // waiting for them (loads complete in issue order for the wait
        // counter) does not wait for the rows, which stream in meanwhile.
        __builtin_amdgcn_sched_barrier(0);
        load_k(k0);
        load_v(k0);
        __builtin_amdgcn_sched_barrier(0);
    }
    float ga[HPW], gb[HPW], av[HPW], bv[HPW];
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
        const int h = wave + hh * kWaves;
        const bool gained = h <= G && (h < G ? a.q_norm : a.k_norm) != nullptr;
        ga[hh] = gained ? bf16_to_f32((uint16_t)gra[hh]) : 1.f;
        gb[hh] = gained ? bf16_to_f32((uint16_t)grb[hh]) : 1.f;
        av[hh] = h <= G ? ar[hh] : 0.f;
        bv[hh] = h <= G ? br[hh] : 0.f;
    }
    float vnew = tid < HD ? vraw : 0.f;
    if (WORDS) {
        for (int it = 0;; ++it) {
            int ok = 1;
#pragma unroll
            for (int hh = 0; hh < HPW; ++hh) {
                const int h = wave + hh * kWaves;
                if (h <= G) {
                    const unsigned long long *x =
                        h < G ? words + (size_t)(qh0 + h) * HD : words + qd + (size_t)g * HD;
                    const unsigned long long wa =
                        __hip_atomic_load(x + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    const unsigned long long wb =
                        __hip_atomic_load(x + lane + HALF, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ok &= (unsigned)(wa >> 32) == epoch && (unsigned)(wb >> 32) == epoch;
                    av[hh] = __uint_as_float((unsigned)wa);
                    bv[hh] = __uint_as_float((unsigned)wb);
                }
            }
            if (tid < HD) {
                const unsigned long long wv = __hip_atomic_load(words + qd + kvd + (size_t)g * HD + tid,
                                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ok &= (unsigned)(wv >> 32) == epoch;
                vnew = __uint_as_float((unsigned)wv);
            }
            if (__syncthreads_and(ok)) break;
            if (it >= (1 << 21)) {
                if (tid == 0) atomicAdd(err, 1u);
                break;
            }
        }
    }
    if (tid < G) {
        st_m[tid] = -INFINITY;
        st_l[tid] = 0.f;
    }
    if (tid < HD) hv[tid] = vnew;
    // RMSNorm (model.rs:111-116) + RoPE (model.rs:117-118), one head per wave.
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
        const int h = wave + hh * kWaves;
        if (h > G) continue;
        float x0 = av[hh], x1 = bv[hh];
        if (h < G ? a.q_norm != nullptr : a.k_norm != nullptr) {
            const float ss = wave_sum_dpp(x0 * x0 + x1 * x1);
            const float sc = 1.0f / sqrtf(ss / (float)HD + a.eps);
            x0 = x0 * (sc * ga[hh]);
            x1 = x1 * (sc * gb[hh]);
        }
        float *x = h < G ? hq + h * HD : hk;
        x[lane] = x0 * cs.x - x1 * cs.y;
        x[lane + HALF] = x1 * cs.x + x0 * cs.y;
    }
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)HD);
    float acc[G][4];
#pragma unroll
    for (int gg = 0; gg < G; ++gg)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[gg][i] = 0.f;
    const long long s1 = s0 + chunk < len ? s0 + chunk : len;
    for (long long c0 = s0; c0 < s1; c0 += ROWS) {
        const int cnt = (int)(s1 - c0 < ROWS ? s1 - c0 : ROWS);
        const bool more = c0 + ROWS < s1;
        // Scores: positions below pos come from the cache, pos itself is the
        // new key. q is read from LDS once per pass, all heads together.
        float qf[G][8];
#pragma unroll
        for (int gg = 0; gg < G; ++gg) lds_row8(hq + gg * HD, sub, qf[gg]);
#pragma unroll
        for (int i = 0; i < NK; ++i) {
            const int j = i * 16 + kq;
            float kf[8];
            R::unpack_k(kr[i], kf);
            if (c0 + j == pos) lds_row8(hk, sub, kf);
#pragma unroll
            for (int gg = 0; gg < G; ++gg) {
                float sc = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) sc = fmaf(qf[gg][e], kf[e], sc);
                sc = row_sum_dpp(sc);
                if (sub == 0 && j < cnt) scores[gg][j] = scale * sc;
            }
        }
        if (more) load_k(c0 + ROWS);
        __syncthreads();
        // Online softmax, one wave per q head.
        if (wave < G) {
            float m = -INFINITY;
            for (int j = lane; j < cnt; j += 64) m = fmaxf(m, scores[wave][j]);
            m = wave_max_dpp(m);
            const float m_old = st_m[wave], m_new = fmaxf(m_old, m);
            float l = 0.f;
            for (int j = lane; j < cnt; j += 64) {
                const float e = expf(scores[wave][j] - m_new);
                scores[wave][j] = e;
                l += e;
            }
            l = wave_sum_dpp(l);
            if (lane == 0) {
                const float al = expf(m_old - m_new);
                st_a[wave] = al;
                st_l[wave] = st_l[wave] * al + l;
                st_m[wave] = m_new;
            }
        }
        __syncthreads();
#pragma unroll
        for (int gg = 0; gg < G; ++gg) {
            const float al = st_a[gg];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[gg][i] *= al;
        }
        // Weights of this lane's keys, eight keys at a time, all of a chunk
        // read before any is used (0 past the context, where the value
        // registers hold rows that are not used).
        const long long fresh = pos - c0 - pv;  // slot * 8 of the key at pos, if this lane holds it
        constexpr int PC = NV < 8 ? NV : 8;
#pragma unroll
        for (int i0 = 0; i0 < NV; i0 += PC) {
            float pw[PC][G];
#pragma unroll
            for (int i = 0; i < PC; ++i)
#pragma unroll
                for (int gg = 0; gg < G; ++gg)
                    pw[i][gg] = (i0 + i) * 8 + pv < cnt ? scores[gg][(i0 + i) * 8 + pv] : 0.f;
#pragma unroll
            for (int i = 0; i < PC; ++i) {
                if ((i0 + i) * 8 + pv < cnt) {
                    float vf[4];
                    R::unpack_v(vr[i0 + i], vf);
                    if (fresh == (i0 + i) * 8) {
                        const float4 n = reinterpret_cast<const float4 *>(hv)[d4];
                        vf[0] = n.x; vf[1] = n.y; vf[2] = n.z; vf[3] = n.w;
                    }
#pragma unroll
                    for (int gg = 0; gg < G; ++gg)
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[gg][e] = fmaf(pw[i][gg], vf[e], acc[gg][e]);
                }
            }
        }
        if (more) load_v(c0 + ROWS);
        __syncthreads();  // scores are rewritten by the next pass
    }
    // The split holding pos appends the new key and value (model.rs:119-120);
    // no block of this launch reads that position from the caches.
    if (append && pos >= s0 && pos < s0 + chunk && tid < HD) {
        store_kv(const_cast<KV *>(kc) + pos * HD + tid, hk[tid]);
        store_kv(const_cast<KV *>(vc) + pos * HD + tid, hv[tid]);
    }
    // Sum the 8 key groups: lanes l and l + 32 of a wave, then the 4 waves.
#pragma unroll
    for (int gg = 0; gg < G; ++gg)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            acc[gg][i] += __shfl_xor(acc[gg][i], 32, 64);
            if (lane < 32) red[gg][wave][d4 * 4 + i] = acc[gg][i];
        }
    __syncthreads();
    const int n_live = (int)((len + chunk - 1) / chunk);  // chunks holding positions
    for (int idx = tid; idx < G * HD; idx += kThreads) {
        const int gg = idx / HD, d = idx % HD;
        const float sm = ((red[gg][0][d] + red[gg][1][d]) + red[gg][2][d]) + red[gg][3][d];
        const long long h = (long long)qh0 + gg;
        if (xw && n_live > 1) {
            chunk_finish(a, h, d, sm, st_m[gg], st_l[gg], xw, n_chunks, split, n_live, epoch, err);
            continue;
        }
        if (a.nsplit == 1) {
            a.out[h * HD + d] = sm / st_l[gg];
        } else {
            const long long slot = h * a.nsplit + split;
            a.part_acc[slot * HD + d] = sm;
            if (d == 0) {
                a.part_ml[slot * 2] = st_m[gg];
                a.part_ml[slot * 2 + 1] = st_l[gg];
            }
        }
    }
}

// Value pairs (dims 2 lane, 2 lane + 1 of a row) as the four-wave attention
// holds them.
template <typename KV> struct VPair;
template <> struct VPair<float> {
    using T = float2;
    __device__ static T load(const float *row, int lane) { return reinterpret_cast<const float2 *>(row)[lane]; }
    __device__ static float2 get(const T &v) { return v; }
};
template <> struct VPair<uint16_t> {
    using T = uint32_t;
    __device__ static T load(const uint16_t *row, int lane) { return reinterpret_cast<const uint32_t *>(row)[lane]; }
    __device__ static float2 get(const T &v) { return make_float2(bf16_lo(v), bf16_hi(v)); }
};

// Attention of one q head h (of KV head g) over one chunk of the cache, rows
// [split * kRows, + kRows) (64 f32 / 128 bf16 positions), by the block's four
// waves with two block barriers. Waves 0, 1 and 2 poll the q, k and v words
// (q and k are normalized and rotated in registers) into LDS; then wave w
// takes a quarter of the rows: its lanes score them in groups of
// 64 / rows-per-wave lanes (each load instruction reads consecutive 16-byte
// chunks of every row), the wave takes the max and sum of its rows with DPP
// reductions and accumulates P.V for two dimensions a lane, each row's weight
// broadcast from the lane that holds it. The four (sum, max, denominator)
// partials merge in wave order and chunk_finish ends the chunk. The cached
// rows, the norm gains and the RoPE row are requested at the start, before
// the words arrive; rows past max_len come from the caches' tail and, like
// every row past the context, are masked.
template <typename KV>
__device__ __forceinline__ void attend_wave4(const StepAttnArgs &a, int g, int h, bool append, int split,
                                             const unsigned long long *words, unsigned epoch, unsigned *err,
                                             unsigned long long *xw, int n_chunks) {
    constexpr int HD = 128, HALF = HD / 2;
    constexpr int ROWS = KvRegs<KV>::kRows;
    constexpr int RW = ROWS / kWaves;         // rows per wave: 16 f32 / 32 bf16
    constexpr int LPR = 64 / RW;              // lanes per row in the scores: 4 / 2
    constexpr int DPL = HD / LPR;             // dims per lane in the scores: 32 / 64
    constexpr int EPV = 16 / (int)sizeof(KV); // elements per 16-byte load
    constexpr int NKL = DPL / EPV;            // 16-byte K loads per lane: 8
    static_assert(LPR == 2 || LPR == 4, "row groups within a DPP quad");
    __shared__ float hq[HD], hk[HD], hv[HD];
    __shared__ float pacc[kWaves][HD], pm[kWaves], pl[kWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int qd = a.n_heads * HD, kvd = a.n_kv_heads * HD;
    const long long max_len = a.head_stride / HD;
    const long long s0 = (long long)split * ROWS;
    const long long pos = *(const __attribute__((address_space(4))) long long *)a.pos;
    const long long len = pos + 1;
    if (s0 >= len) return;  // a chunk past the context (uniform over the block)
    const KV *kc = reinterpret_cast<const KV *>(a.k_cache) + (size_t)g * a.head_stride;
    const KV *vc = reinterpret_cast<const KV *>(a.v_cache) + (size_t)g * a.head_stride;
    const long long r0 = s0 + wave * RW;                  // this wave's first row
    const long long rb = r0 < max_len ? r0 : max_len - 1;  // where its loads start
    const int sr = lane / LPR, sj = lane % LPR;           // score row of the lane, slice of it
    // K: 16-byte chunk i * LPR + sj of the row, i < NKL (each load instruction
    // reads LPR consecutive chunks of every row); V: dims 2 lane, 2 lane + 1.
    uint4 kr[NKL];
    typename VPair<KV>::T vr[RW];
    {
        const uint4 *kp = reinterpret_cast<const uint4 *>(kc + (rb + sr) * HD);
#pragma unroll
        for (int i = 0; i < NKL; ++i) kr[i] = kp[i * LPR + sj];
#pragma unroll
        for (int r = 0; r < RW; ++r) vr[r] = VPair<KV>::load(vc + (rb + r) * HD, lane);
    }
    const float2 cs = reinterpret_cast<const float2 *>(a.rope + pos * HD)[lane];
    const float gq0 = a.q_norm ? bf16_to_f32(a.q_norm[lane]) : 1.f;
    const float gq1 = a.q_norm ? bf16_to_f32(a.q_norm[lane + HALF]) : 1.f;
    const float gk0 = a.k_norm ? bf16_to_f32(a.k_norm[lane]) : 1.f;
    const float gk1 = a.k_norm ? bf16_to_f32(a.k_norm[lane + HALF]) : 1.f;
    // The raw q (head h), k and v (KV head g) rows from the epoch words, one
    // row a wave (waves 0, 1, 2), normalized and rotated in registers.
    if (wave < 3) {
        const unsigned long long *src = wave == 0   ? words + (size_t)h * HD
                                        : wave == 1 ? words + qd + (size_t)g * HD
                                                    : words + qd + kvd + (size_t)g * HD;
        unsigned long long wa, wb;
        for (int it = 0;; ++it) {
            wa = __hip_atomic_load(src + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            wb = __hip_atomic_load(src + lane + HALF, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const bool ok = (unsigned)(wa >> 32) == epoch && (unsigned)(wb >> 32) == epoch;
            if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
            if (it >= (1 << 21)) {
                if (lane == 0) atomicAdd(err, 1u);
                break;
            }
        }
        float x0 = __uint_as_float((unsigned)wa), x1 = __uint_as_float((unsigned)wb);
        float *dst = wave == 0 ? hq : wave == 1 ? hk : hv;
        if (wave < 2) {
            // RMSNorm (model.rs:111-116) + RoPE (model.rs:117-118).
            if (wave == 0 ? a.q_norm != nullptr : a.k_norm != nullptr) {
                const float ss = wave_sum_dpp(x0 * x0 + x1 * x1);
                const float sc = 1.0f / sqrtf(ss / (float)HD + a.eps);
                x0 = x0 * (sc * (wave == 0 ? gq0 : gk0));
                x1 = x1 * (sc * (wave == 0 ? gq1 : gk1));
            }
            dst[lane] = x0 * cs.x - x1 * cs.y;
            dst[lane + HALF] = x1 * cs.x + x0 * cs.y;
        } else {
            dst[lane] = x0;
            dst[lane + HALF] = x1;
        }
    }
    __syncthreads();
    // Scores: row r0 + sr, dims [sj * DPL, + DPL); the row at pos is the new key.
    const long long row = r0 + sr;
    const bool fresh = row == pos;
    float sc = 0.f;
#pragma unroll
    for (int i = 0; i < NKL; ++i) {
        float kf[EPV];
        if (EPV == 8) {
            unpack8(kr[i], kf);
        } else {
            kf[0] = __uint_as_float(kr[i].x);
            kf[1] = __uint_as_float(kr[i].y);
            kf[2] = __uint_as_float(kr[i].z);
            kf[3] = __uint_as_float(kr[i].w);
        }
        const int c = (i * LPR + sj) * EPV;  // first dim of the chunk
        if (fresh) {
#pragma unroll
            for (int e = 0; e < EPV; ++e) kf[e] = hk[c + e];
        }
        const float *qs = hq + c;
#pragma unroll
        for (int e = 0; e < EPV; ++e) sc = fmaf(qs[e], kf[e], sc);
    }
    sc += dpp_get<0xB1>(sc, 0.f);                // quad_perm [1,0,3,2]
    if (LPR == 4) sc += dpp_get<0x4E>(sc, 0.f);  // quad_perm [2,3,0,1]
    const bool valid = row < len;
    const float s = valid ? sc * (1.0f / sqrtf((float)HD)) : -INFINITY;
    // Softmax statistics of the wave's rows.
    const float m = wave_max_dpp(s);
    const float p = valid ? expf(s - m) : 0.f;  // m is finite when any row is valid
    const float l = wave_sum_dpp(sj == 0 ? p : 0.f);
    // P.V: dims 2 lane, 2 lane + 1; the row at pos is the new value. Rows
    // past the context hold stale bits (NaN among them): their values are
    // replaced by 0 (their weights are 0 already), so that the loop runs
    // without branches; adding 0 * 0 leaves the sums as they were.
    const float2 hv2 = reinterpret_cast<const float2 *>(hv)[lane];
    float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const float pr = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), r * LPR));
        float2 v = VPair<KV>::get(vr[r]);
        const bool fr = r0 + r == pos, live = r0 + r < len;
        v.x = fr ? hv2.x : (live ? v.x : 0.f);
        v.y = fr ? hv2.y : (live ? v.y : 0.f);
        acc0 = fmaf(pr, v.x, acc0);
        acc1 = fmaf(pr, v.y, acc1);
    }
    pacc[wave][2 * lane] = acc0;
    pacc[wave][2 * lane + 1] = acc1;
    if (lane == 0) {
        pm[wave] = m;
        pl[wave] = l;
    }
    // The group's first head appends the new key and value (model.rs:119-120);
    // no block of this launch reads that position from the caches.
    if (append && wave == 0 && pos >= s0 && pos < s0 + ROWS) {
        store_kv(const_cast<KV *>(kc) + pos * HD + lane, hk[lane]);
        store_kv(const_cast<KV *>(kc) + pos * HD + lane + HALF, hk[lane + HALF]);
        store_kv(const_cast<KV *>(vc) + pos * HD + lane, hv[lane]);
        store_kv(const_cast<KV *>(vc) + pos * HD + lane + HALF, hv[lane + HALF]);
    }
    __syncthreads();
    if (tid < HD) {
        // Merge the waves in order (a wave with no row in the context adds nothing).
        const float mx = fmaxf(fmaxf(pm[0], pm[1]), fmaxf(pm[2], pm[3]));
        float num = 0.f, den = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float e = pm[w] == -INFINITY ? 0.f : expf(pm[w] - mx);
            num = fmaf(pacc[w][tid], e, num);
            den = fmaf(pl[w], e, den);
        }
        const int n_live = (int)((len + ROWS - 1) / ROWS);
        chunk_finish(a, h, tid, num, mx, den, xw, n_chunks, split, n_live, epoch, err);
    }
}

}  // namespace

}  // namespace th
