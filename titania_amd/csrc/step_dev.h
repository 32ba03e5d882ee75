// Device code of the decode-step kernels: the GEMV input builder, row tables,
// the fused launch's attention of one q head over one chunk of the cache, and
// the streaming split attention of one KV head's q heads for long contexts.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <type_traits>

#include "device_util.h"
#include "fused.h"
#include "step.h"

namespace th {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

// The block's input x = a (+ b) in registers, NV float4 of each a thread,
// and the RMSNorm gains of those elements.
template <int NV>
struct InputRegs {
    float4 va[NV], vb[NV];
    uint2 vg[NV];
};

// Issues the loads of the block's input vectors a (and b, if not null).
template <int NV>
__device__ __forceinline__ void load_input(InputRegs<NV> &in, const float *a, const float *b, int n) {
    const int tid = threadIdx.x, n4 = n >> 2;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int i = tid + k * kThreads;
        if (i < n4) {
            in.va[k] = reinterpret_cast<const float4 *>(a)[i];
            if (b) in.vb[k] = reinterpret_cast<const float4 *>(b)[i];
        }
    }
}

// Issues the loads of the bf16 RMSNorm gains g of the block's input.
template <int NV>
__device__ __forceinline__ void load_gain(InputRegs<NV> &in, const uint16_t *g, int n) {
    const int tid = threadIdx.x, n4 = n >> 2;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int i = tid + k * kThreads;
        if (i < n4) in.vg[k] = reinterpret_cast<const uint2 *>(g)[i];
    }
}

// Builds the block's f32 input in LDS from the loaded vectors: x = a (+ b
// when has_b), optionally RMSNorm'd with the loaded gains (model/cpu.rs:85-94);
// block 0 keeps the un-normalized sum in x_out. All loads are issued before
// any is used, so the input costs one memory round trip rather than one per
// loop iteration.
template <bool NORM, int NV>
__device__ __forceinline__ void finish_input(InputRegs<NV> &in, float *xs, bool has_b, int n, float eps,
                                             float *x_out, float *red) {
    const int tid = threadIdx.x;
    const int n4 = n >> 2;
    float4 *va = in.va;
    const float4 *vb = in.vb;
    const uint2 *vg = in.vg;
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int i = tid + k * kThreads;
        if (i < n4) {
            float4 v = va[k];
            if (has_b) {
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

// load_input and finish_input in one: the input's loads, then its use.
template <bool NORM, int NV>
__device__ __forceinline__ void build_input(float *xs, const float *a, const float *b, int n, const uint16_t *g,
                                            float eps, float *x_out, float *red) {
    InputRegs<NV> in;
    load_input(in, a, b, n);
    if (NORM) load_gain(in, g, n);
    finish_input<NORM>(in, xs, b != nullptr, n, eps, x_out, red);
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

// Cached positions one attention block of the fused q/k/v + attention launch
// takes (a register pass of rows: 64 f32 or 128 bf16, 64 KB of keys and
// values).
template <typename KV> struct KvRegs;
template <> struct KvRegs<float> {
    static constexpr int kRows = 64;
};
template <> struct KvRegs<uint16_t> {
    static constexpr int kRows = 128;
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

// Cached rows of the streaming attention as 16-byte chunks: 4 f32 or 8 bf16
// values each.
template <typename KV> struct StreamKV;
template <> struct StreamKV<float> {
    static constexpr int EPC = 4;  // elements per chunk
    __device__ static void unpack(const uint4 &k, float f[EPC]) {
        f[0] = __uint_as_float(k.x); f[1] = __uint_as_float(k.y);
        f[2] = __uint_as_float(k.z); f[3] = __uint_as_float(k.w);
    }
};
template <> struct StreamKV<uint16_t> {
    static constexpr int EPC = 8;
    __device__ static void unpack(const uint4 &k, float f[EPC]) { unpack8(k, f); }
};

// Sum over the 16 lanes of each DPP row, left in every lane of the row.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_get<0xB1>(v, 0.f);   // quad_perm [1,0,3,2]
    v += dpp_get<0x4E>(v, 0.f);   // quad_perm [2,3,0,1]
    v += dpp_get<0x141>(v, 0.f);  // row_half_mirror: the other quad of the half-row
    v += dpp_get<0x140>(v, 0.f);  // row_mirror: the other half of the row
    return v;
}

// The fields the streaming attention reads before the position is known,
// without WORDS: the caches' bases and head stride (max_len * head_dim), the
// raw q/k/v rows, the q/k RMSNorm gains (or null) and the head counts.
struct StreamHead {
    const void *k_cache, *v_cache;
    const float *qkv;
    const uint16_t *q_norm, *k_norm;
    int head_stride;
    int n_heads, n_kv_heads;
};

// Attention of one KV head's G q heads over the positions [s0, s0 + chunk)
// of the context (s0 = split * chunk) by one block, for contexts past the
// fused launch's reach. The cached rows stream through registers in passes
// of 32 positions (8 a wave), the next pass's rows requested before the
// current pass's arithmetic, so that every wave keeps a pass of loads in
// flight. Each wave scores and weighs only its own rows of every pass, with
// an online softmax of its own (no block barrier between passes); the four
// waves merge once, at the end, into the split's (sum, max, denominator)
// partials for launch_attn_combine, or into the output with one split.
//
// Layout: the 16 lanes of DPP row r (r < 4) take the wave's rows r and r + 4
// of a pass; a lane holds 8 dims of each (its 16-byte chunks sub + 16 i of
// the row's key and value), so that each load instruction reads whole
// 256-byte spans of four rows. A row's dot product is summed over its 16
// lanes with DPP (every lane gets it), and a lane weighs its own value dims
// by its own rows' weights. A lane keeps its 8 dims of q (scaled by
// log2(e) / sqrt(head_dim): the softmax runs in base 2) and of each head's
// weighted sums in registers; the rows' sums merge once, at the end. The raw
// q/k/v come from a.qkv, or (WORDS) from the (value | epoch << 32) words of
// the same launch's GEMV blocks, polled (bounded) after the first pass's
// rows are requested. Without WORDS, for f32 caches, `e` (preloaded) gives
// what the first requests need: the raw q/k/v rows, the gains and the first
// pass's rows go out before the position is read, a device value behind the kernel
// arguments whose round trip then overlaps their flight. With WORDS the rows
// wait for the position: requested any earlier they compete with the same
// launch's GEMV blocks, whose words the attention waits for.
template <int G, typename KV, bool WORDS>
__device__ __forceinline__ void attend_stream(const StepAttnArgs &a, int g, int split, long long chunk,
                                              const unsigned long long *words, unsigned epoch, unsigned *err,
                                              const StreamHead *e = nullptr) {
    using T = StreamKV<KV>;
    constexpr int HD = 128, HALF = HD / 2, LPR = 16, EPC = T::EPC;
    constexpr int RS = 2;                   // rows a lane takes each pass
    constexpr int RW = 4 * RS;              // rows a wave takes each pass
    constexpr int PASS = RW * kWaves;       // rows a block takes each pass
    constexpr int NC = HD / EPC / LPR;      // 16-byte chunks of a row a lane holds (2 f32 / 1 bf16)
    constexpr int DL = NC * EPC;            // dims a lane holds: 8
    constexpr int HPW = (G + 1 + kWaves - 1) / kWaves;  // heads (q..., k) a wave normalizes
    static_assert(DL == 8 && PASS <= kStepKvTailRows, "8 dims a lane; a pass within the caches' tail");
    // The early requests (below) for f32 caches only: with bf16 caches they
    // measured slower (Qwen3-4B at 8192 positions 2.084 -> 2.098 ms a step).
    constexpr bool EARLY = !WORDS && std::is_same<KV, float>::value;
    __shared__ float hq[G * HD], hk[HD], hv[HD];
    // Each DPP row's weighted sums, per wave, head and dim.
    __shared__ float4 red[kWaves][4][G][HD / 4];
    __shared__ float wm[kWaves][G], wl[kWaves][G];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sub = lane % LPR, drow = lane / LPR;
    const int qd = (EARLY ? e->n_heads : a.n_heads) * HD, kvd = (EARLY ? e->n_kv_heads : a.n_kv_heads) * HD;
    const KV *kc = EARLY ? reinterpret_cast<const KV *>(e->k_cache) + (size_t)g * e->head_stride
                         : reinterpret_cast<const KV *>(a.k_cache) + (size_t)g * a.head_stride;
    const KV *vc = EARLY ? reinterpret_cast<const KV *>(e->v_cache) + (size_t)g * e->head_stride
                         : reinterpret_cast<const KV *>(a.v_cache) + (size_t)g * a.head_stride;
    constexpr int ROWB = HD * (int)sizeof(KV);  // bytes a row
    uint4 ka[RS][NC], kb[RS][NC], va[RS][NC], vb[RS][NC];
    // RMSNorm gains of this wave's heads (q heads 0..G-1, then k), and the
    // raw q/k rows (without WORDS).
    uint32_t gra[HPW], grb[HPW];
    float ar[HPW], br[HPW], vraw = 0.f;
    uint16_t g16a[HPW], g16b[HPW];  // EARLY: the gains as loaded
    if constexpr (EARLY) {
        // The gains, the raw rows (from e->qkv), then the first pass's rows,
        // whatever the position: a split's start lies inside the caches (rows
        // past them would come from the allocation's tail of kStepKvTailRows
        // rows, and rows past the context are ignored below).
#pragma unroll
        for (int hh = 0; hh < HPW; ++hh) {
            const int h = min(wave + hh * kWaves, G);
            const uint16_t *gain = h < G ? e->q_norm : e->k_norm;
            const uint16_t *gp = gain ? gain : reinterpret_cast<const uint16_t *>(e->qkv);
            g16a[hh] = gp[lane];
            g16b[hh] = gp[lane + HALF];
            const float *x = h < G ? e->qkv + (size_t)(g * G + h) * HD : e->qkv + qd + (size_t)g * HD;
            ar[hh] = x[lane];
            br[hh] = x[lane + HALF];
        }
        vraw = e->qkv[qd + kvd + (size_t)g * HD + (tid & (HD - 1))];
        const int c0 = split * (int)chunk;
        const bool live = c0 < e->head_stride / HD;
        const __amdgpu_buffer_rsrc_t sk =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<KV *>(kc), 0, live ? 0x7fffffff : 0, kBufferRsrcWord3);
        const __amdgpu_buffer_rsrc_t sv =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<KV *>(vc), 0, live ? 0x7fffffff : 0, kBufferRsrcWord3);
        const int o = (wave * RW + drow) * ROWB + sub * 16, base = c0 * ROWB;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < RS; ++r)
#pragma unroll
            for (int i = 0; i < NC; ++i) {
                const th_u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(sk, o + 4 * r * ROWB + i * LPR * 16, base, 0);
                ka[r][i] = make_uint4(x.x, x.y, x.z, x.w);
            }
#pragma unroll
        for (int r = 0; r < RS; ++r)
#pragma unroll
            for (int i = 0; i < NC; ++i) {
                const th_u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(sv, o + 4 * r * ROWB + i * LPR * 16, base, 0);
                va[r][i] = make_uint4(x.x, x.y, x.z, x.w);
            }
        __builtin_amdgcn_sched_barrier(0);
    }
    // Positions fit 32 bits (a cache of head_dim floats a row is far smaller
    // than 2^31 rows): 32-bit scalar arithmetic keeps the loop's bounds in
    // scalar registers.
    const int pos = (int)*(const __attribute__((address_space(4))) long long *)a.pos;
    const int len = pos + 1;
    const int s0 = split * (int)chunk;
    const int s1 = s0 + (int)chunk < len ? s0 + (int)chunk : len;
    if (s0 >= s1) {
        if constexpr (EARLY) {
            // The raw rows and the first pass's rows count as used here too,
            // as loaded (no arithmetic on them, which the compiler would
            // hoist above the branch with a wait): otherwise it sinks their
            // loads into the other path, behind the position's read. The
            // 16-bit gains are left out: their widening would be hoisted.
#pragma unroll
            for (int hh = 0; hh < HPW; ++hh) asm volatile("" ::"v"(ar[hh]), "v"(br[hh]));
            asm volatile("" ::"v"(vraw));
#pragma unroll
            for (int r = 0; r < RS; ++r)
#pragma unroll
                for (int i = 0; i < NC; ++i)
                    asm volatile("" ::"v"(ka[r][i].x), "v"(ka[r][i].y), "v"(ka[r][i].z), "v"(ka[r][i].w),
                                 "v"(va[r][i].x), "v"(va[r][i].y), "v"(va[r][i].z), "v"(va[r][i].w));
        }
        // No positions here: empty partials (finite zeros, max -inf) for the combine.
        for (int idx = tid; idx < G * HD; idx += kThreads) {
            const long long slot = (long long)(g * G + idx / HD) * a.nsplit + split;
            a.part_acc[slot * HD + idx % HD] = 0.f;
            if (idx % HD == 0) {
                a.part_ml[slot * 2] = -INFINITY;
                a.part_ml[slot * 2 + 1] = 0.f;
            }
        }
        return;
    }
    // Buffer loads from the head's base (scalar registers): a lane's offsets
    // within a pass are fixed, the pass's start is a scalar offset, so the
    // loads need no 64-bit address registers.
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<KV *>(kc), 0, 0x7fffffff, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<KV *>(vc), 0, 0x7fffffff, kBufferRsrcWord3);
    const int ofs = (wave * RW + drow) * ROWB + sub * 16;
    // A request with no pass left goes through descriptors of no records:
    // the same instructions (so that every wait counts the same requests),
    // answered with zeros and no memory access, so the block ends without
    // waiting for rows it would not use.
    const __amdgpu_buffer_rsrc_t nk =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<KV *>(kc), 0, 0, kBufferRsrcWord3);
    const __amdgpu_buffer_rsrc_t nv =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<KV *>(vc), 0, 0, kBufferRsrcWord3);
    auto load = [&](uint4 (&k)[RS][NC], uint4 (&v)[RS][NC], int c0, bool live = true) {
        const __amdgpu_buffer_rsrc_t sk = live ? rk : nk, sv = live ? rv : nv;
        const int base = c0 * ROWB;
#pragma unroll
        for (int r = 0; r < RS; ++r)
#pragma unroll
            for (int i = 0; i < NC; ++i) {
                const th_u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(sk, ofs + 4 * r * ROWB + i * LPR * 16, base, 0);
                k[r][i] = make_uint4(x.x, x.y, x.z, x.w);
            }
#pragma unroll
        for (int r = 0; r < RS; ++r)
#pragma unroll
            for (int i = 0; i < NC; ++i) {
                const th_u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(sv, ofs + 4 * r * ROWB + i * LPR * 16, base, 0);
                v[r][i] = make_uint4(x.x, x.y, x.z, x.w);
            }
    };
    if (WORDS) load(ka, va, s0);  // the words come long after the rows
    const float2 cs = reinterpret_cast<const float2 *>(a.rope + (size_t)pos * HD)[lane];
    // Unless EARLY, the gains and, from a.qkv, the raw rows: loaded with no
    // branch and used only after the rows are requested, so that no wait for
    // them comes first.
    if constexpr (!EARLY) {
#pragma unroll
        for (int hh = 0; hh < HPW; ++hh) {
            const int h = min(wave + hh * kWaves, G);
            const uint16_t *gain = h < G ? a.q_norm : a.k_norm;
            const uint16_t *gp = gain ? gain : reinterpret_cast<const uint16_t *>(a.rope);
            gra[hh] = gp[lane];
            grb[hh] = gp[lane + HALF];
            ar[hh] = br[hh] = 0.f;
            if (!WORDS) {
                const float *x = h < G ? a.qkv + (size_t)(g * G + h) * HD : a.qkv + qd + (size_t)g * HD;
                ar[hh] = x[lane];
                br[hh] = x[lane + HALF];
            }
        }
        if (!WORDS) {
            vraw = a.qkv[qd + kvd + (size_t)g * HD + (tid & (HD - 1))];
            __builtin_amdgcn_sched_barrier(0);
            load(ka, va, s0);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    float av[HPW], bv[HPW];
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
        const int h = wave + hh * kWaves;
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
                    const unsigned long long *x = h < G ? words + (size_t)(g * G + h) * HD : words + qd + (size_t)g * HD;
                    const unsigned long long w0 = __hip_atomic_load(x + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    const unsigned long long w1 =
                        __hip_atomic_load(x + lane + HALF, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ok &= (unsigned)(w0 >> 32) == epoch && (unsigned)(w1 >> 32) == epoch;
                    av[hh] = __uint_as_float((unsigned)w0);
                    bv[hh] = __uint_as_float((unsigned)w1);
                }
            }
            if (tid < HD) {
                const unsigned long long w2 = __hip_atomic_load(words + qd + kvd + (size_t)g * HD + tid,
                                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ok &= (unsigned)(w2 >> 32) == epoch;
                vnew = __uint_as_float((unsigned)w2);
            }
            if (__syncthreads_and(ok)) break;
            if (it >= (1 << 21)) {
                if (tid == 0) atomicAdd(err, 1u);
                break;
            }
        }
    }
    if (tid < HD) hv[tid] = vnew;
    // RMSNorm (model.rs:111-116) + RoPE (model.rs:117-118), one head a wave.
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
        const int h = wave + hh * kWaves;
        if (h > G) continue;
        float x0 = av[hh], x1 = bv[hh];
        if (h < G ? a.q_norm != nullptr : a.k_norm != nullptr) {
            const float ss = wave_sum_dpp(x0 * x0 + x1 * x1);
            const float sc = 1.0f / sqrtf(ss / (float)HD + a.eps);
            x0 = x0 * (sc * bf16_to_f32(EARLY ? g16a[hh] : (uint16_t)gra[hh]));
            x1 = x1 * (sc * bf16_to_f32(EARLY ? g16b[hh] : (uint16_t)grb[hh]));
        }
        float *x = h < G ? hq + h * HD : hk;
        x[lane] = x0 * cs.x - x1 * cs.y;
        x[lane + HALF] = x1 * cs.x + x0 * cs.y;
    }
    __syncthreads();
    // The lane's dims of q, scaled into the base-2 domain: scores come out as
    // s * log2(e) / sqrt(HD), so that each weight is one v_exp_f32.
    const float scale2 = 1.4426950408889634f / sqrtf((float)HD);
    float q[G][DL];
#pragma unroll
    for (int gg = 0; gg < G; ++gg)
#pragma unroll
        for (int i = 0; i < NC; ++i)
#pragma unroll
            for (int e = 0; e < EPC; ++e) q[gg][i * EPC + e] = scale2 * hq[gg * HD + (sub + LPR * i) * EPC + e];
    // m: the wave's running maximum (uniform); l: the lane's running sum of
    // its rows' weights; acc: its 8 dims' weighted sums of its rows' values.
    float m[G], l[G], acc[G][DL];
#pragma unroll
    for (int gg = 0; gg < G; ++gg) {
        m[gg] = -INFINITY;
        l[gg] = 0.f;
#pragma unroll
        for (int e = 0; e < DL; ++e) acc[gg][e] = 0.f;
    }
    // One pass over rows c0.. (the new key and value at pos from LDS: the
    // caches do not hold them yet).
    auto pass = [&](const uint4 (&k)[RS][NC], const uint4 (&v)[RS][NC], int c0) {
        const bool has_pos = c0 <= pos && pos < c0 + PASS;  // uniform over the block
        const bool whole = c0 + PASS <= s1;                  // uniform: every row in the context
        float kf[RS][DL], vf[RS][DL];
        bool valid[RS];
#pragma unroll
        for (int r = 0; r < RS; ++r) {
            const int row = c0 + wave * RW + drow + 4 * r;
            valid[r] = row < s1;
#pragma unroll
            for (int i = 0; i < NC; ++i) {
                T::unpack(k[r][i], kf[r] + i * EPC);
                T::unpack(v[r][i], vf[r] + i * EPC);
            }
            if (has_pos && row == pos) {
                // The new key and value (their cache row is stale).
#pragma unroll
                for (int i = 0; i < NC; ++i)
#pragma unroll
                    for (int e = 0; e < EPC; ++e) {
                        kf[r][i * EPC + e] = hk[(sub + LPR * i) * EPC + e];
                        vf[r][i * EPC + e] = hv[(sub + LPR * i) * EPC + e];
                    }
            }
            if (!whole && !valid[r]) {
                // Rows past the context hold stale bits (NaN among them):
                // their weight is 0, and their value is replaced by 0 too.
#pragma unroll
                for (int e = 0; e < DL; ++e) vf[r][e] = 0.f;
            }
        }
        // Scores of the lane's two rows for every head: independent chains.
        float sc[RS][G];
#pragma unroll
        for (int r = 0; r < RS; ++r)
#pragma unroll
            for (int gg = 0; gg < G; ++gg) {
                float t = 0.f;
#pragma unroll
                for (int e = 0; e < DL; ++e) t = fmaf(q[gg][e], kf[r][e], t);
                sc[r][gg] = t;
            }
#pragma unroll
        for (int r = 0; r < RS; ++r)
#pragma unroll
            for (int gg = 0; gg < G; ++gg) sc[r][gg] = row16_sum(sc[r][gg]);
        if (!whole) {
            // Rows past the context: score -inf (weight 0).
#pragma unroll
            for (int r = 0; r < RS; ++r)
#pragma unroll
                for (int gg = 0; gg < G; ++gg) sc[r][gg] = valid[r] ? sc[r][gg] : -INFINITY;
        }
#pragma unroll
        for (int gg = 0; gg < G; ++gg) {
            // The wave's maximum over its 8 rows (scores are finite or -inf).
            float mx = sc[0][gg];
#pragma unroll
            for (int r = 1; r < RS; ++r) mx = max_nn(mx, sc[r][gg]);
            mx = rows_max_nn(mx);
            if (mx > m[gg]) {  // uniform: rescale only when the maximum rises
                const float alpha = m[gg] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[gg] - mx);
                l[gg] *= alpha;
#pragma unroll
                for (int e = 0; e < DL; ++e) acc[gg][e] *= alpha;
                m[gg] = mx;
            }
            // exp2(-inf - m) = 0 for the rows past the context (m is finite:
            // the wave has seen a row of the context by now, or all its rows
            // so far are past it and m, mx and every score are -inf).
            const float mm = m[gg] == -INFINITY ? 0.f : m[gg];
#pragma unroll
            for (int r = 0; r < RS; ++r) {
                const float p = __builtin_amdgcn_exp2f(sc[r][gg] - mm);
                l[gg] += p;
#pragma unroll
                for (int e = 0; e < DL; ++e) acc[gg][e] = fmaf(p, vf[r][e], acc[gg][e]);
            }
        }
    };
    // Passes two at a time through the two register sets: the next pass's
    // rows are requested before this pass's arithmetic, unconditionally (with
    // no pass left, through the descriptors of no records), so that the wait
    // for a pass's rows never waits for the next pass's.
    for (int c0 = s0; c0 < s1; c0 += 2 * PASS) {
        const int c1 = c0 + PASS;
        load(kb, vb, c1 < s1 ? c1 : c0, c1 < s1);
        pass(ka, va, c0);
        if (c1 >= s1) break;
        load(ka, va, c1 + PASS < s1 ? c1 + PASS : c1, c1 + PASS < s1);
        pass(kb, vb, c1);
    }
    // The split holding pos appends the new key and value (model.rs:119-120);
    // no block of this launch reads that position from the caches.
    if (pos >= s0 && pos < s0 + (int)chunk && tid < HD) {
        store_kv(const_cast<KV *>(kc) + (size_t)pos * HD + tid, hk[tid]);
        store_kv(const_cast<KV *>(vc) + (size_t)pos * HD + tid, hv[tid]);
    }
    // Every lane of a DPP row holds its rows' weighted sums for its dims: the
    // rows go to LDS; the weight sums over the wave's rows (each lane holds
    // its two rows', the same in every lane of the DPP row). The waves and
    // rows merge in order, the maxima back in base e.
#pragma unroll
    for (int gg = 0; gg < G; ++gg) {
        const float ls = rows_sum(l[gg]);
#pragma unroll
        for (int i = 0; i < NC; ++i)
#pragma unroll
            for (int e4 = 0; e4 < EPC / 4; ++e4)
                red[wave][drow][gg][((sub + LPR * i) * EPC) / 4 + e4] =
                    make_float4(acc[gg][i * EPC + 4 * e4], acc[gg][i * EPC + 4 * e4 + 1],
                                acc[gg][i * EPC + 4 * e4 + 2], acc[gg][i * EPC + 4 * e4 + 3]);
        if (lane == 0) {
            wm[wave][gg] = m[gg] * 0.6931471805599453f;
            wl[wave][gg] = ls;
        }
    }
    __syncthreads();
    for (int idx = tid; idx < G * HD; idx += kThreads) {
        const int gg = idx / HD, d = idx % HD;
        const float mx = fmaxf(fmaxf(wm[0][gg], wm[1][gg]), fmaxf(wm[2][gg], wm[3][gg]));
        float num = 0.f, den = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float e = wm[w][gg] == -INFINITY ? 0.f : expf(wm[w][gg] - mx);
            const float *r = reinterpret_cast<const float *>(&red[w][0][gg][0]) + d;
            constexpr int RSTR = G * HD;  // floats between DPP rows
            const float sw = ((r[0] + r[RSTR]) + r[2 * RSTR]) + r[3 * RSTR];
            num = fmaf(sw, e, num);
            den = fmaf(wl[w][gg], e, den);
        }
        const long long h = (long long)g * G + gg;
        if (a.nsplit == 1) {
            a.out[h * HD + d] = num / den;
        } else {
            const long long slot = h * a.nsplit + split;
            a.part_acc[slot * HD + d] = num;
            if (d == 0) {
                a.part_ml[slot * 2] = mx;
                a.part_ml[slot * 2 + 1] = den;
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
    // The launch's chunks must cover the context (the host picks a launch of
    // fewer chunks than the caches hold only while they do): past them rows
    // would go unread, so the head's first chunk flags it.
    if (split == 0 && threadIdx.x == 0 && len > (long long)n_chunks * ROWS) atomicAdd(err, kStepReachError);
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
