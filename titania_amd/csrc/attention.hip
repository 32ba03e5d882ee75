// Device::attention (model/cpu.rs:113-149): causal grouped-query attention over
// key/value caches, as split-K flash decoding.
//
// One block handles one (token, KV head, split of the sequence); every query
// head that shares the KV head is processed in the same block, so each cached
// key and value row is read once per block. A split walks its positions in
// sub-chunks of up to 256 whose scores sit in LDS, keeping a running max, sum
// of exponentials and unnormalized accumulator (online softmax). With one split
// the block writes the normalized output; otherwise it writes its partial and
// a combine pass merges the splits by log-sum-exp rescaling.
//
// The split ranges are derived on the device from the token's context length,
// so a launch of fixed shape serves any position; the position may come from
// device memory, which lets one captured decode step replay at every position.
#include "common.h"
#include "device_util.h"
#include "gemm.h"

namespace th {

constexpr int kAttnMaxGroup = 8;   // query heads per KV head
constexpr int kAttnSub = 256;      // positions scored per sub-chunk
constexpr size_t kAttnTileMin = 8; // tokens from which a launch uses the matrix-core kernel
constexpr size_t kMKTiles = 32;    // positions per key tile of the one-head-a-block kernel
constexpr int kMQT = 64;           // tokens per block of that kernel
constexpr int kGqaRows = 128, kGqaKeys = 64;  // (token, head) rows a block, keys a tile: GQA kernel
constexpr size_t kRowPassH = 64;    // positions a pass of the few-token kernel (kRowPass)

template <typename KV>
__device__ __forceinline__ void load8(const KV *p, float f[8]);

template <>
__device__ __forceinline__ void load8<float>(const float *p, float f[8]) {
    float4 a = reinterpret_cast<const float4 *>(p)[0], b = reinterpret_cast<const float4 *>(p)[1];
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}

template <>
__device__ __forceinline__ void load8<uint16_t>(const uint16_t *p, float f[8]) {
    unpack8(*reinterpret_cast<const uint4 *>(p), f);
}

__device__ __forceinline__ float load1(const float *p) { return *p; }
__device__ __forceinline__ float load1(const uint16_t *p) { return bf16_to_f32(*p); }

template <int HD, typename KV>
__global__ __launch_bounds__(256) void attn_split_kernel(AttnKernelArgs a) {
    constexpr int LPK = HD / 8;      // lanes per key row (8 elements each)
    constexpr int KPW = 64 / LPK;    // key rows per wave per step
    constexpr int KPB = 4 * KPW;     // key rows per block per step
    constexpr int NP = 256 / HD;     // thread groups splitting the value rows

    __shared__ float scores[kAttnMaxGroup][kAttnSub];
    __shared__ float red[kAttnMaxGroup][256];
    __shared__ float stat_m[kAttnMaxGroup], stat_l[kAttnMaxGroup], alpha[kAttnMaxGroup];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int split = blockIdx.x % a.nsplit;
    const int g = (blockIdx.x / a.nsplit) % a.n_kv_heads;
    const long long t = blockIdx.x / (a.nsplit * a.n_kv_heads);
    const int G = a.group;
    const long long pos = a.pos_dev ? *a.pos_dev : a.pos;
    const long long len = pos + t + 1;  // the token attends up to its own position
    const long long chunk = ((len + a.nsplit - 1) / a.nsplit + 15) / 16 * 16;
    const long long s0 = (long long)split * chunk;
    const long long s1 = s0 + chunk < len ? s0 + chunk : len;

    const KV *kb = reinterpret_cast<const KV *>(a.k) + (long long)g * a.head_stride;
    const KV *vb = reinterpret_cast<const KV *>(a.v) + (long long)g * a.head_stride;

    // This lane's 8 elements of every query head in the group.
    const int sub = lane % LPK;
    float qf[kAttnMaxGroup][8];
#pragma unroll
    for (int gg = 0; gg < kAttnMaxGroup; ++gg) {
        if (gg < G) {
            const float *qh = a.q + ((t * a.n_heads) + (long long)g * G + gg) * HD + sub * 8;
            load8<float>(qh, qf[gg]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) qf[gg][i] = 0.f;
        }
    }
    if (tid < kAttnMaxGroup) {
        stat_m[tid] = -INFINITY;
        stat_l[tid] = 0.f;
    }

    const int d = tid % HD, part = tid / HD;
    float acc[kAttnMaxGroup];
#pragma unroll
    for (int gg = 0; gg < kAttnMaxGroup; ++gg) acc[gg] = 0.f;

    for (long long c0 = s0; c0 < s1; c0 += kAttnSub) {
        const int cnt = (int)(s1 - c0 < kAttnSub ? s1 - c0 : kAttnSub);
        // Scores q . k_j * scale.
        for (int j0 = 0; j0 < cnt; j0 += KPB) {
            const int j = j0 + wave * KPW + lane / LPK;
            const bool valid = j < cnt;
            float kf[8];
            if (valid) {
                load8<KV>(kb + (c0 + j) * a.pos_stride + sub * 8, kf);
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) kf[i] = 0.f;
            }
#pragma unroll
            for (int gg = 0; gg < kAttnMaxGroup; ++gg) {
                if (gg < G) {
                    float dd = 0.f;
#pragma unroll
                    for (int i = 0; i < 8; ++i) dd = fmaf(qf[gg][i], kf[i], dd);
                    dd = group_sum<LPK>(dd);
                    if (valid && sub == 0) scores[gg][j] = a.scale * dd;
                }
            }
        }
        __syncthreads();
        // Per query head: new running max, exponentials in place, running sum.
        for (int gg = wave; gg < G; gg += 4) {
            float m = -INFINITY;
            for (int j = lane; j < cnt; j += 64) m = fmaxf(m, scores[gg][j]);
            m = wave_max(m);
            const float m_old = stat_m[gg];
            const float m_new = fmaxf(m_old, m);
            float l = 0.f;
            for (int j = lane; j < cnt; j += 64) {
                float p = expf(scores[gg][j] - m_new);
                scores[gg][j] = p;
                l += p;
            }
            l = wave_sum(l);
            if (lane == 0) {
                const float al = expf(m_old - m_new);
                alpha[gg] = al;
                stat_l[gg] = stat_l[gg] * al + l;
                stat_m[gg] = m_new;
            }
        }
        __syncthreads();
        // acc = acc * alpha + sum of p_j * v_j; thread (part, d) takes every NP-th position.
#pragma unroll
        for (int gg = 0; gg < kAttnMaxGroup; ++gg)
            if (gg < G) acc[gg] *= alpha[gg];
        for (int j = part; j < cnt; j += NP) {
            float v = load1(vb + (c0 + j) * a.pos_stride + d);
#pragma unroll
            for (int gg = 0; gg < kAttnMaxGroup; ++gg)
                if (gg < G) acc[gg] = fmaf(scores[gg][j], v, acc[gg]);
        }
        __syncthreads();  // scores and alpha are rewritten by the next sub-chunk
    }

    __syncthreads();  // the statistics are complete (also when the split is empty)
    if (NP > 1) {
#pragma unroll
        for (int gg = 0; gg < kAttnMaxGroup; ++gg)
            if (gg < G) red[gg][tid] = acc[gg];
        __syncthreads();
        if (part == 0) {
#pragma unroll
            for (int gg = 0; gg < kAttnMaxGroup; ++gg) {
                if (gg < G) {
                    float s = red[gg][d];
                    for (int p = 1; p < NP; ++p) s += red[gg][p * HD + d];
                    acc[gg] = s;
                }
            }
        }
    }
    if (part != 0) return;

    for (int gg = 0; gg < G; ++gg) {
        const long long h = (long long)g * G + gg;
        if (a.nsplit == 1) {
            a.out[(t * a.n_heads + h) * HD + d] = acc[gg] / stat_l[gg];
        } else {
            const long long slot = (t * a.n_heads + h) * a.nsplit + split;
            a.part_acc[slot * HD + d] = acc[gg];
            if (d == 0) {
                a.part_ml[slot * 2] = stat_m[gg];
                a.part_ml[slot * 2 + 1] = stat_l[gg];
            }
        }
    }
}

// Attention of a few tokens (decode) with head_dim 128: one block per (token,
// KV head, split of the positions); a split walks its positions in passes of
// kRowPass rows whose keys and values every thread requests into registers at
// once (the next pass's keys while this pass's softmax and P.V run). Keys:
// thread t holds a quarter (32 dimensions) of row t / 4; the G query heads
// come from LDS as broadcasts, and a quad of lanes sums a row's score. Values:
// thread t holds dimensions 2 (t % 64) + {0, 1} of rows 16 (t / 64) + [0, 16)
// and accumulates p . v for each head; the four row groups are summed in LDS
// at the end. Scores, probabilities and the per-head statistics live in LDS.
constexpr int kRowPass = (int)kRowPassH;

template <typename KV>
__global__ __launch_bounds__(256) void attn_rows_kernel(AttnKernelArgs a) {
    constexpr int HD = 128, P = kRowPass, G_MAX = kAttnMaxGroup;
    constexpr bool F32 = sizeof(KV) == 4;
    constexpr int KV8 = 16 / sizeof(KV);  // elements of a 16-byte load
    __shared__ __align__(16) float qs[G_MAX][HD];
    __shared__ float sc[G_MAX][P];
    __shared__ __align__(16) float red[4][G_MAX][HD];
    __shared__ float st_m[G_MAX], st_l[G_MAX], st_a[G_MAX];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int split = blockIdx.x % a.nsplit;
    const int g = (blockIdx.x / a.nsplit) % a.n_kv_heads;
    const long long t = blockIdx.x / (a.nsplit * a.n_kv_heads);
    const int G = a.group;
    const long long pos = a.pos_dev ? *a.pos_dev : a.pos;
    const long long len = pos + t + 1;  // the token attends up to its own position
    const long long chunk = ((len + a.nsplit - 1) / a.nsplit + P - 1) / P * P;
    const long long s0 = (long long)split * chunk;
    const long long s1 = s0 + chunk < len ? s0 + chunk : len;
    const KV *kb = reinterpret_cast<const KV *>(a.k) + (long long)g * a.head_stride;
    const KV *vb = reinterpret_cast<const KV *>(a.v) + (long long)g * a.head_stride;

    const int kr = tid >> 2, kq = tid & 3;     // key row, quarter of its dimensions
    const int vd = 2 * (tid & 63), vq = tid >> 6;  // value dimension pair, row group
    KV kreg[32];
    float vreg[16][2];
    auto fetch_k = [&](long long c0) {
        const long long r = c0 + kr < s1 ? c0 + kr : s1 - 1;  // rows past the split repeat its last row
        const uint4 *src = reinterpret_cast<const uint4 *>(kb + r * a.pos_stride + 32 * kq);
#pragma unroll
        for (int i = 0; i < 32 / KV8; ++i) reinterpret_cast<uint4 *>(kreg)[i] = src[i];
    };
    auto fetch_v = [&](long long c0) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const long long r0 = c0 + 16 * vq + i, r = r0 < s1 ? r0 : s1 - 1;
            const KV *src = vb + r * a.pos_stride + vd;
            if constexpr (F32) {
                const float2 v = *reinterpret_cast<const float2 *>(src);
                vreg[i][0] = v.x;
                vreg[i][1] = v.y;
            } else {
                const uint32_t w = *reinterpret_cast<const uint32_t *>(src);
                vreg[i][0] = bf16_lo(w);
                vreg[i][1] = bf16_hi(w);
            }
        }
    };
    if (s0 < s1) {
        fetch_k(s0);
        fetch_v(s0);
    }
    for (int i = tid; i < G * HD; i += 256)
        qs[i / HD][i % HD] = a.q[((t * a.n_heads) + (long long)g * G + i / HD) * HD + i % HD];
    if (tid < G_MAX) {
        st_m[tid] = -INFINITY;
        st_l[tid] = 0.f;
    }
    float acc[G_MAX][2];
#pragma unroll
    for (int gg = 0; gg < G_MAX; ++gg) acc[gg][0] = acc[gg][1] = 0.f;
    __syncthreads();

    for (long long c0 = s0; c0 < s1; c0 += P) {
        // Scores of row c0 + kr for every head: a quad of lanes sums the quarters.
        float kf[32];
#pragma unroll
        for (int j = 0; j < 32; ++j) kf[j] = F32 ? (float)kreg[j] : bf16_to_f32((uint16_t)kreg[j]);
        const bool row_in = c0 + kr < s1;
#pragma unroll
        for (int gg = 0; gg < G_MAX; ++gg) {
            if (gg < G) {
                const float4 *qv = reinterpret_cast<const float4 *>(&qs[gg][32 * kq]);
                float d = 0.f;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float4 q4 = qv[j];
                    d = fmaf(q4.x, kf[4 * j], d);
                    d = fmaf(q4.y, kf[4 * j + 1], d);
                    d = fmaf(q4.z, kf[4 * j + 2], d);
                    d = fmaf(q4.w, kf[4 * j + 3], d);
                }
                d += dpp_get<0xB1>(d, 0.f);
                d += dpp_get<0x4E>(d, 0.f);
                if (kq == 0) sc[gg][kr] = row_in ? a.scale * d : -INFINITY;
            }
        }
        if (c0 + P < s1) fetch_k(c0 + P);
        __syncthreads();
        // Online softmax per head, one wave per head.
        for (int gg = wave; gg < G; gg += 4) {
            const float v = sc[gg][lane];
            const float m_old = st_m[gg];
            const float m_new = fmaxf(m_old, wave_max_dpp(v));
            const float p = v == -INFINITY ? 0.f : expf(v - m_new);
            sc[gg][lane] = p;
            const float l = wave_sum_dpp(p);
            if (lane == 0) {
                const float al = m_old == -INFINITY ? 0.f : expf(m_old - m_new);
                st_a[gg] = al;
                st_l[gg] = st_l[gg] * al + l;
                st_m[gg] = m_new;
            }
        }
        __syncthreads();
        // acc = acc * alpha + p . v over this thread's 16 rows.
#pragma unroll
        for (int gg = 0; gg < G_MAX; ++gg) {
            if (gg < G) {
                const float al = st_a[gg];
                float x0 = acc[gg][0] * al, x1 = acc[gg][1] * al;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const float p = sc[gg][16 * vq + i];
                    x0 = fmaf(p, vreg[i][0], x0);
                    x1 = fmaf(p, vreg[i][1], x1);
                }
                acc[gg][0] = x0;
                acc[gg][1] = x1;
            }
        }
        if (c0 + P < s1) fetch_v(c0 + P);
        __syncthreads();  // sc and st_a are rewritten by the next pass
    }
#pragma unroll
    for (int gg = 0; gg < G_MAX; ++gg)
        if (gg < G) *reinterpret_cast<float2 *>(&red[vq][gg][vd]) = make_float2(acc[gg][0], acc[gg][1]);
    __syncthreads();
    for (int i = tid; i < G * HD; i += 256) {
        const int gg = i / HD, d = i % HD;
        const float v = red[0][gg][d] + red[1][gg][d] + red[2][gg][d] + red[3][gg][d];
        const long long h = (long long)g * G + gg;
        if (a.nsplit == 1) {
            a.out[(t * a.n_heads + h) * HD + d] = v / st_l[gg];
        } else {
            const long long slot = (t * a.n_heads + h) * a.nsplit + split;
            a.part_acc[slot * HD + d] = v;
            if (d == 0) {
                a.part_ml[slot * 2] = st_m[gg];
                a.part_ml[slot * 2 + 1] = st_l[gg];
            }
        }
    }
}

// Merges the splits of one (token, head): rescales each split's sum and
// accumulator by exp(m_split - m_max); empty splits (m = -inf) add nothing.
// Every split's statistics and accumulator rows are read in parallel (threads
// over splits, then over (dimension, group of splits)), not one after another.
constexpr int kCombineThreads = 256, kMaxSplits = 256;

// gy is gridDim.y, passed as an argument so that it arrives preloaded with
// the others (the grid's size is otherwise one more fetch before the first
// loads can be addressed).
__global__ __launch_bounds__(kCombineThreads) void attn_combine_kernel(float *__restrict__ out,
                                                                      const float *__restrict__ part_acc,
                                                                      const float *__restrict__ part_ml, int nsplit,
                                                                      int hd, int gy, uint16_t *__restrict__ hi,
                                                                      uint16_t *__restrict__ lo) {
    constexpr int kPre = 16;  // accumulator rows a thread requests up front
    __shared__ float w[kMaxSplits];
    __shared__ float red[kCombineThreads / 64];
    __shared__ float acc_red[kCombineThreads];
    const long long th = blockIdx.x;  // token * n_heads + head
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *ml = part_ml + th * nsplit * 2;
    // This block's dimensions [dlo, dlo + dw) (gy blocks share a head), in
    // groups of splits: thread t takes dimension dlo + t % dw of the splits
    // s = t / dw, + groups, ...
    const int dw = hd / gy, dlo = (int)blockIdx.y * dw;
    const int groups = dw < kCombineThreads ? kCombineThreads / dw : 1;
    // With one pass over the dimensions and at most kPre splits a thread
    // (every launch of the decode step), the accumulator rows are requested
    // with the statistics, so the merge waits for one memory round trip
    // instead of three; the sums run in the same order either way (Qwen3-0.6B
    // decode after a 4096-token prompt: 0.925 -> 0.903 ms a step).
    const bool pre = dw <= kCombineThreads && nsplit <= kCombineThreads && nsplit <= kPre * groups;
    float2 st = make_float2(-INFINITY, 0.f);
    float pacc[kPre];
    if (pre) {
        if (tid < nsplit) st = reinterpret_cast<const float2 *>(ml)[tid];
        const int dd = tid % dw, grp = tid / dw;
        const float *pa = part_acc + th * nsplit * hd + dlo + dd;
#pragma unroll
        for (int k = 0; k < kPre; ++k) {
            const int s = grp + k * groups;
            pacc[k] = grp < groups && s < nsplit ? pa[(size_t)s * hd] : 0.f;
        }
    }
    float m = -INFINITY;
    if (pre) m = st.x;
    else
        for (int s = tid; s < nsplit; s += kCombineThreads) m = fmaxf(m, ml[2 * s]);
    m = wave_max_dpp(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float l = 0.f;
    if (pre) {
        if (tid < nsplit) {
            const float ws = st.x != -INFINITY ? expf(st.x - m) : 0.f;
            w[tid] = ws;
            l = st.y * ws;
        }
    } else {
        for (int s = tid; s < nsplit; s += kCombineThreads) {
            const float ms = ml[2 * s];
            const float ws = ms != -INFINITY ? expf(ms - m) : 0.f;
            w[s] = ws;
            l += ml[2 * s + 1] * ws;
        }
    }
    l = wave_sum_dpp(l);
    if (lane == 0) red[wave] = l;
    __syncthreads();
    l = ((red[0] + red[1]) + red[2]) + red[3];
    for (int d0 = 0; d0 < dw; d0 += kCombineThreads) {
        const int dd = d0 + tid % dw, grp = tid / dw, d = dlo + dd;
        float acc = 0.f;
        if (pre) {
            if (grp < groups) {
#pragma unroll
                for (int k = 0; k < kPre; ++k) {
                    const int s = grp + k * groups;
                    if (s < nsplit) acc += pacc[k] * w[s];
                }
            }
        } else if (dd < dw && grp < groups) {
            const float *pa = part_acc + th * nsplit * hd + d;
#pragma unroll 8
            for (int s = grp; s < nsplit; s += groups) acc += pa[(size_t)s * hd] * w[s];
        }
        acc_red[tid] = acc;
        __syncthreads();
        if (grp == 0 && dd < dw) {
            float sum = 0.f;
            for (int gi = 0; gi < groups; ++gi) sum += acc_red[gi * dw + tid % dw];
            if (hi)
                split_bf16(sum / l, hi[th * hd + d], lo[th * hd + d]);
            else
                out[th * hd + d] = sum / l;
        }
        __syncthreads();
    }
}

// The same merge with one wave per (token, head), for many pairs of few
// splits (prefill): lane s holds split s's statistics, each lane HD / 64
// dimensions of the accumulators, walked over the splits in order.
template <int HD>
__global__ __launch_bounds__(256) void attn_combine_wave_kernel(float *__restrict__ out,
                                                                const float *__restrict__ part_acc,
                                                                const float *__restrict__ part_ml, int nsplit,
                                                                long long heads, uint16_t *__restrict__ hi,
                                                                uint16_t *__restrict__ lo) {
    constexpr int D = HD / 64;
    const long long th = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (th >= heads) return;
    // The first kPre splits' partials are requested with the (max,
    // denominator) pairs, so that the merge waits for one round trip.
    constexpr int kPre = 8;
    const float *pa = part_acc + th * nsplit * HD + lane * D;
    float pre[kPre][D];
#pragma unroll
    for (int sp = 0; sp < kPre; ++sp)
        if (sp < nsplit)
#pragma unroll
            for (int d = 0; d < D; ++d) pre[sp][d] = pa[(size_t)sp * HD + d];
    float ms = -INFINITY, ls = 0.f;
    if (lane < nsplit) {
        const float2 v = reinterpret_cast<const float2 *>(part_ml + th * nsplit * 2)[lane];
        ms = v.x;
        ls = v.y;
    }
    const float m = wave_max_dpp(ms);
    const float ws = ms != -INFINITY ? expf(ms - m) : 0.f;
    const float l = wave_sum_dpp(ls * ws);
    float acc[D];
#pragma unroll
    for (int d = 0; d < D; ++d) acc[d] = 0.f;
#pragma unroll
    for (int sp = 0; sp < kPre; ++sp) {
        if (sp < nsplit) {
            const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ws), sp));
#pragma unroll
            for (int d = 0; d < D; ++d) acc[d] += pre[sp][d] * w;
        }
    }
    for (int sp = kPre; sp < nsplit; ++sp) {
        const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ws), sp));
#pragma unroll
        for (int d = 0; d < D; ++d) acc[d] += pa[(size_t)sp * HD + d] * w;
    }
    const long long o = th * HD + lane * D;
#pragma unroll
    for (int d = 0; d < D; ++d) {
        if (hi)
            split_bf16(acc[d] / l, hi[o + d], lo[o + d]);
        else
            out[o + d] = acc[d] / l;
    }
}

// The same merge for few (token, head) pairs of at most kCombineLaneSplits
// splits (decode): one wave per (pair, 8 dimensions), with no block barrier
// among the waves. Lane s holds the statistics of splits s and s + 64; lane
// 8 q + d accumulates dimension d over the splits q, q + 8, q + 16, ...,
// whose accumulator rows it requests together with the statistics, so that
// the merge waits for one memory round trip. The weights pass through LDS in
// that order (the wave's own writes, then its reads); the eight groups' sums
// combine with a DPP rotation and permlane swaps. Slices of 8 dimensions
// measured faster than 16 (twice the waves, half the loads a lane) at the
// Qwen3-0.6B shape, 4096 positions: 0.7455 -> 0.7376 ms a step; 4 were
// slower (0.7472). A wave reads 32 bytes of each split's 512-byte partial
// row, so a head's 16 waves share its 128-byte lines: with `xcd` (heads a
// multiple of 8) they are numbered so that all of them run on one XCD
// (blocks go to the 8 XCDs in turn), whose L2 then fetches each line once
// rather than each XCD that reads it (Qwen3-4B at 8192 positions 2.2024-
// 2.2105 -> 2.1904-2.2005 ms, Qwen3-0.6B at 4096 0.7372 -> 0.7352 ms).
constexpr int kCombineLaneSplits = 128;

__global__ __launch_bounds__(64) void attn_combine_lanes_kernel(float *__restrict__ out,
                                                                const float *__restrict__ part_acc,
                                                                const float *__restrict__ part_ml, int nsplit, int hd,
                                                                uint16_t *__restrict__ hi, uint16_t *__restrict__ lo,
                                                                int xcd) {
    constexpr int NG = 8, K = kCombineLaneSplits / NG;  // groups of splits; splits a lane
    __shared__ float4 wsh[NG][K / 4];
    const int slices = hd / 8;
    long long th;
    int sl;
    if (xcd) {
        const int j = (int)blockIdx.x / 8;
        th = (long long)(j / slices) * 8 + blockIdx.x % 8;
        sl = j % slices;
    } else {
        th = blockIdx.x / slices;
        sl = (int)(blockIdx.x % slices);
    }
    const int lane = threadIdx.x, grp = lane >> 3;
    const int d = sl * 8 + (lane & 7);
    const float2 *ml = reinterpret_cast<const float2 *>(part_ml + th * nsplit * 2);
    const float *pa = part_acc + th * nsplit * hd + d;
    const float2 st0 = lane < nsplit ? ml[lane] : make_float2(-INFINITY, 0.f);
    const float2 st1 = lane + 64 < nsplit ? ml[lane + 64] : make_float2(-INFINITY, 0.f);
    float pacc[K];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int s = grp + NG * k;
        pacc[k] = s < nsplit ? pa[(size_t)s * hd] : 0.f;
    }
    const float m = wave_max_dpp(fmaxf(st0.x, st1.x));
    // Splits past nsplit and empty splits (max -inf) weigh 0; their
    // accumulators are zeros.
    const float w0 = st0.x != -INFINITY ? expf(st0.x - m) : 0.f;
    const float w1 = st1.x != -INFINITY ? expf(st1.x - m) : 0.f;
    const float l = wave_sum_dpp(st0.y * w0 + st1.y * w1);
    float *wf = reinterpret_cast<float *>(&wsh[0][0]);
    wf[(lane % NG) * K + lane / NG] = w0;
    wf[((lane + 64) % NG) * K + (lane + 64) / NG] = w1;
    __syncthreads();
    float acc = 0.f;
#pragma unroll
    for (int k4 = 0; k4 < K / 4; ++k4) {
        const float4 w = wsh[grp][k4];
        acc = fmaf(pacc[4 * k4], w.x, acc);
        acc = fmaf(pacc[4 * k4 + 1], w.y, acc);
        acc = fmaf(pacc[4 * k4 + 2], w.z, acc);
        acc = fmaf(pacc[4 * k4 + 3], w.w, acc);
    }
    acc += dpp_get<0x128>(acc, 0.f);
    acc = rows_sum(acc);
    if (grp == 0) {
        if (hi)
            split_bf16(acc / l, hi[th * hd + d], lo[th * hd + d]);
        else
            out[th * hd + d] = acc / l;
    }
}

int attention_splits(size_t n, size_t n_heads, size_t n_kv_heads, size_t max_len, size_t head_dim) {
    // Several tokens on the matrix cores: split the keys until the launch has
    // about 512 blocks (two a CU), keeping at least two 64-key tiles a split,
    // at most 8 splits (each split adds partials for the combine to read, and
    // one split needs no combine launch at all). Splitting on to about 1024
    // blocks was slower: 9.71 against 9.26 ms for a 2048-token Qwen3-0.6B
    // prefill, 205.7 against 202.5 ms for 8192 tokens of the Qwen3-4B shape.
    if (head_dim == 128 && n >= kAttnTileMin) {
        const size_t group = n_kv_heads ? n_heads / n_kv_heads : 0;
        const bool gqa = group >= 1 && group <= 8 && 8 % group == 0 && group * n_kv_heads == n_heads;
        const size_t qt = gqa ? kGqaRows / group : kMQT;
        const size_t blocks = (n + qt - 1) / qt * (gqa ? n_kv_heads : n_heads);
        const size_t tiles = (max_len + kGqaKeys - 1) / kGqaKeys;
        size_t ns = 1;
        while (ns < 8 && blocks * ns < 512 && tiles >= 4 * ns) ns *= 2;
        return (int)ns;
    }
    // Few tokens, head_dim 128 (attn_rows_kernel): one split per pass of 64
    // positions, at most 256 splits (longer contexts walk several passes a
    // split).
    if (head_dim == 128 && n_kv_heads && n_heads / n_kv_heads <= (size_t)kAttnMaxGroup)
        return (int)std::max<size_t>(1, std::min<size_t>((max_len + kRowPassH - 1) / kRowPassH, 256));
    // Otherwise split the positions until the launch has about 1024 blocks
    // (a block walks its positions one 256-row pass at a time, so short
    // splits in many blocks keep more rows in flight), each split covering at
    // least 64 positions, at most 256 splits.
    size_t blocks_per_split = n * n_kv_heads;
    size_t want = (1024 + blocks_per_split - 1) / blocks_per_split;
    size_t cap = (max_len + 63) / 64;
    size_t s = std::min(want, cap);
    return (int)std::max<size_t>(1, std::min<size_t>(s, 256));
}

size_t attention_scratch(size_t n, size_t n_heads, size_t head_dim, int nsplit) {
    if (nsplit <= 1) return 0;
    return n * n_heads * (size_t)nsplit * (head_dim + 2);
}

hipError_t launch_attn_combine(hipStream_t s, float *out, const float *part_acc, const float *part_ml, size_t heads,
                               int nsplit, int hd, uint16_t *hi, uint16_t *lo) {
    if (nsplit > kMaxSplits || (!hi != !lo)) return hipErrorInvalidValue;
    if (heads >= 1024 && nsplit <= 64 && (hd == 64 || hd == 128 || hd == 256)) {
        const dim3 grid((unsigned)((heads + 3) / 4));
        switch (hd) {
        case 64: attn_combine_wave_kernel<64><<<grid, 256, 0, s>>>(out, part_acc, part_ml, nsplit, heads, hi, lo); break;
        case 128: attn_combine_wave_kernel<128><<<grid, 256, 0, s>>>(out, part_acc, part_ml, nsplit, heads, hi, lo); break;
        default: attn_combine_wave_kernel<256><<<grid, 256, 0, s>>>(out, part_acc, part_ml, nsplit, heads, hi, lo); break;
        }
        return hipGetLastError();
    }
    if (nsplit <= kCombineLaneSplits && hd % 16 == 0) {
        attn_combine_lanes_kernel<<<(unsigned)(heads * (size_t)(hd / 8)), 64, 0, s>>>(out, part_acc, part_ml, nsplit,
                                                                                        hd, hi, lo, heads % 8 == 0);
        return hipGetLastError();
    }
    // Few (token, head) pairs (decode): their dimensions spread over several
    // blocks each, at least 16 a block, so that the launch fills the chip.
    unsigned ysplit = 1;
    while (heads * ysplit < 256 && hd % (int)(ysplit * 2) == 0 && hd / (int)(ysplit * 2) >= 16) ysplit *= 2;
    attn_combine_kernel<<<dim3((unsigned)heads, ysplit), dim3(kCombineThreads), 0, s>>>(out, part_acc, part_ml,
                                                                                         nsplit, hd, (int)ysplit, hi,
                                                                                         lo);
    return hipGetLastError();
}

__device__ __forceinline__ float4 load4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ float4 load4(const uint16_t *p) {
    const uint2 w = *reinterpret_cast<const uint2 *>(p);
    return make_float4(bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y));
}

// Prefill on the matrix cores (head_dim 128): a flash attention with one
// block per (tile of 64 consecutive tokens, query head, key split), 16 tokens
// per wave. Key/value rows walk through LDS 32 positions at a time (loaded
// into registers one tile ahead). Each wave forms S = Q K^T for its 16
// queries, applies the causal mask and the online softmax along its 16-lane
// rows, passes P through LDS into the A-operand layout and adds P V into
// 16 x 128 f32 accumulators. The products run on v_mfma_f32_16x16x32_bf16:
// every f32 operand is split into bf16 terms x = hi + lo (split_bf16; q and
// the probabilities always, an f32 cache's keys and values too; a bf16 cache
// is exact in hi) and a product is the sum of the hi*hi, hi*lo and lo*hi
// terms (relative error ~2^-16), accumulated in f32. Keys are staged in LDS
// as bf16 rows, values transposed (dimension x key) so that a lane's eight
// keys of one dimension are one 16-byte read. Layout of 16x16x32: lane l
// holds A[l%16][8(l/16)+i], B[8(l/16)+i][l%16] and D[4(l/16)+e][l%16].
constexpr int kMKT = (int)kMKTiles;
typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float row_max16(float v) {
    v = fmaxf(v, dpp_get<0xB1>(v, -INFINITY));
    v = fmaxf(v, dpp_get<0x4E>(v, -INFINITY));
    v = fmaxf(v, dpp_get<0x124>(v, -INFINITY));
    v = fmaxf(v, dpp_get<0x128>(v, -INFINITY));
    return v;
}

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;

__device__ __forceinline__ void split8(const float *f, uint4 &hi, uint4 &lo) {
    uint2 h0, l0, h1, l1;
    split_bf16x4(make_float4(f[0], f[1], f[2], f[3]), h0, l0);
    split_bf16x4(make_float4(f[4], f[5], f[6], f[7]), h1, l1);
    hi = make_uint4(h0.x, h0.y, h1.x, h1.y);
    lo = make_uint4(l0.x, l0.y, l1.x, l1.y);
}

__device__ __forceinline__ bf16x8_t as_bf8(const uint4 &v) { return __builtin_bit_cast(bf16x8_t, v); }

template <typename KV>
__global__ __launch_bounds__(256) void attn_bf16_kernel(AttnKernelArgs a, int n) {
    constexpr bool F32 = sizeof(KV) == 4;
    constexpr int HD = 128, KT = kMKT;                       // dims, keys per tile
    constexpr int KSB = HD + 8, VTS = KT + 8, PS = KT + 4;   // LDS row strides (bf16, bf16, f32)
    __shared__ uint4 ksh[KT * KSB / 8], ksl[F32 ? KT * KSB / 8 : 1];
    __shared__ uint4 vth[HD * VTS / 8], vtl[F32 ? HD * VTS / 8 : 1];
    __shared__ __align__(16) float ps[4][16 * PS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lk = lane >> 4;
    const int h = blockIdx.y, g = h / a.group;
    const int t0 = blockIdx.x * kMQT;
    const int nq = n - t0 < kMQT ? n - t0 : kMQT;
    const long long pos = a.pos_dev ? *a.pos_dev : a.pos;
    // Q of query li of the wave, dims 32 c + 8 lk + [0, 8), as bf16 hi / lo.
    const int tq = t0 + wave * 16 + li;
    uint4 qh[HD / 32], ql[HD / 32];
    {
        const float *qp = a.q + ((long long)(tq < n ? tq : 0) * a.n_heads + h) * HD + 8 * lk;
#pragma unroll
        for (int c = 0; c < HD / 32; ++c) {
            float f[8];
            const float4 x0 = *reinterpret_cast<const float4 *>(qp + 32 * c);
            const float4 x1 = *reinterpret_cast<const float4 *>(qp + 32 * c + 4);
            f[0] = x0.x; f[1] = x0.y; f[2] = x0.z; f[3] = x0.w;
            f[4] = x1.x; f[5] = x1.y; f[6] = x1.z; f[7] = x1.w;
            if (tq >= n)
#pragma unroll
                for (int e = 0; e < 8; ++e) f[e] = 0.f;
            split8(f, qh[c], ql[c]);
        }
    }
    const KV *kb = reinterpret_cast<const KV *>(a.k) + (long long)g * a.head_stride;
    const KV *vb = reinterpret_cast<const KV *>(a.v) + (long long)g * a.head_stride;
    const long long last = pos + t0 + nq - 1;           // the block's last query position
    const long long wlast = pos + t0 + wave * 16 + 15;  // this wave's last query position
    const long long ntiles = last / KT + 1, z = blockIdx.z;
    const long long kt0 = z * ntiles / a.nsplit, kt1 = (z + 1) * ntiles / a.nsplit;
    floatx4 o[HD / 16];
    float m[4], l[4];
#pragma unroll
    for (int d = 0; d < HD / 16; ++d) o[d] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        m[r] = -INFINITY;
        l[r] = 0.f;
    }
    // Staging: thread t loads key t / 8, dims 16 (t % 8) + [0, 16) of K, and
    // keys 8 (t / 64) + [0, 8) of V at dims 2 (t % 64), + 1 (each load
    // instruction of a wave reads consecutive bytes of a row). Positions past
    // the block's last query read as 0.
    const int kkey = tid / 8, kd0 = (tid % 8) * 16, vd = 2 * (tid % 64), vk0 = 8 * (tid / 64);
    float kraw[16], vraw[8][2];
    auto fetch = [&](long long c0) {
        const long long pk = c0 + kkey;
#pragma unroll
        for (int e = 0; e < 16; e += 4) {
            const float4 x = pk <= last ? load4(kb + pk * a.pos_stride + kd0 + e) : make_float4(0.f, 0.f, 0.f, 0.f);
            kraw[e] = x.x; kraw[e + 1] = x.y; kraw[e + 2] = x.z; kraw[e + 3] = x.w;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const long long pv = c0 + vk0 + j;
            float2 v = make_float2(0.f, 0.f);
            if (pv <= last) {
                if (F32) {
                    v = *reinterpret_cast<const float2 *>(reinterpret_cast<const float *>(vb) + pv * a.pos_stride + vd);
                } else {
                    const uint32_t w =
                        *reinterpret_cast<const uint32_t *>(reinterpret_cast<const uint16_t *>(vb) + pv * a.pos_stride + vd);
                    v = make_float2(bf16_lo(w), bf16_hi(w));
                }
            }
            vraw[j][0] = v.x;
            vraw[j][1] = v.y;
        }
    };
    const long long cend = kt1 * KT;
    if (kt0 < kt1) fetch(kt0 * KT);
    for (long long c0 = kt0 * KT; c0 < cend; c0 += KT) {
        __syncthreads();  // the previous tile is consumed
        {
            uint4 hi, lo;
#pragma unroll
            for (int e = 0; e < 16; e += 8) {
                split8(kraw + e, hi, lo);
                ksh[(kkey * KSB + kd0 + e) / 8] = hi;
                if (F32) ksl[(kkey * KSB + kd0 + e) / 8] = lo;
            }
#pragma unroll
            for (int dd = 0; dd < 2; ++dd) {
                float f[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) f[j] = vraw[j][dd];
                split8(f, hi, lo);
                vth[((vd + dd) * VTS + vk0) / 8] = hi;
                if (F32) vtl[((vd + dd) * VTS + vk0) / 8] = lo;
            }
        }
        __syncthreads();
        if (c0 + KT < cend) fetch(c0 + KT);
        if (c0 > wlast) continue;  // every query of this wave precedes the tile
        // S for keys c0 + [0, 16) and c0 + [16, 32).
        floatx4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < HD / 32; ++c) {
            const int off = 32 * c + 8 * lk;
            const bf16x8_t qhc = as_bf8(qh[c]), qlc = as_bf8(ql[c]);
            const bf16x8_t k0 = as_bf8(ksh[(li * KSB + off) / 8]), k1 = as_bf8(ksh[((16 + li) * KSB + off) / 8]);
            s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qhc, k0, s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qhc, k1, s1, 0, 0, 0);
            s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qlc, k0, s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qlc, k1, s1, 0, 0, 0);
            if (F32) {
                const bf16x8_t k0l = as_bf8(ksl[(li * KSB + off) / 8]), k1l = as_bf8(ksl[((16 + li) * KSB + off) / 8]);
                s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qhc, k0l, s0, 0, 0, 0);
                s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qhc, k1l, s1, 0, 0, 0);
            }
        }
        // Causal mask and online softmax of rows 4 lk + r (this lane: keys li, 16 + li).
        float al[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int qi = wave * 16 + 4 * lk + r;  // query within the block
            const long long qp = pos + t0 + qi;
            const bool in = qi < nq;
            const float v0 = in && c0 + li <= qp ? a.scale * s0[r] : -INFINITY;
            const float v1 = in && c0 + 16 + li <= qp ? a.scale * s1[r] : -INFINITY;
            const float mn = fmaxf(m[r], row_max16(fmaxf(v0, v1)));
            const float p0 = v0 == -INFINITY ? 0.f : expf(v0 - mn);
            const float p1 = v1 == -INFINITY ? 0.f : expf(v1 - mn);
            al[r] = m[r] == -INFINITY ? 0.f : expf(m[r] - mn);
            l[r] = l[r] * al[r] + row_sum_dpp(p0 + p1);
            m[r] = mn;
            ps[wave][(4 * lk + r) * PS + li] = p0;
            ps[wave][(4 * lk + r) * PS + 16 + li] = p1;
        }
#pragma unroll
        for (int d = 0; d < HD / 16; ++d)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[d][r] *= al[r];
        // P in the A-operand layout: query li, keys 8 lk + [0, 8) (same wave:
        // LDS stays in order).
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        uint4 ph, pl;
        {
            const float4 x0 = *reinterpret_cast<const float4 *>(&ps[wave][li * PS + 8 * lk]);
            const float4 x1 = *reinterpret_cast<const float4 *>(&ps[wave][li * PS + 8 * lk + 4]);
            const float f[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            split8(f, ph, pl);
        }
        const bf16x8_t pha = as_bf8(ph), pla = as_bf8(pl);
#pragma unroll
        for (int d = 0; d < HD / 16; ++d) {
            const int vo = ((d * 16 + li) * VTS + 8 * lk) / 8;
            const bf16x8_t vh = as_bf8(vth[vo]);
            o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pha, vh, o[d], 0, 0, 0);
            o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pla, vh, o[d], 0, 0, 0);
            if (F32) o[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pha, as_bf8(vtl[vo]), o[d], 0, 0, 0);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int qi = wave * 16 + 4 * lk + r;
        if (qi >= nq) continue;
        const long long th = (long long)(t0 + qi) * a.n_heads + h;
        if (a.nsplit == 1 && a.out_hi) {
#pragma unroll
            for (int d = 0; d < HD / 16; ++d)
                split_bf16(o[d][r] / l[r], a.out_hi[th * HD + li + d * 16], a.out_lo[th * HD + li + d * 16]);
        } else if (a.nsplit == 1) {
            float *op = a.out + th * HD + li;
#pragma unroll
            for (int d = 0; d < HD / 16; ++d) op[d * 16] = o[d][r] / l[r];
        } else {
            const long long slot = th * a.nsplit + z;
            float *op = a.part_acc + slot * HD + li;
#pragma unroll
            for (int d = 0; d < HD / 16; ++d) op[d * 16] = o[d][r];
            if (li == 0) {
                a.part_ml[slot * 2] = m[r];
                a.part_ml[slot * 2 + 1] = l[r];
            }
        }
    }
}

// Prefill attention with the keys and values of a KV group shared by its G
// query heads: one block per (tile of 128 / G tokens, KV head, key split),
// 128 (token, head) rows a block, NW waves of 128 / NW rows, each as sets of
// 16 rows. Keys walk through LDS 64 at a time. Each wave forms S^T = K Q^T
// (keys down, rows across) on v_mfma_f32_16x16x32_bf16, so that the D layout
// leaves a lane sixteen keys of one row: the causal mask, the online softmax
// (base 2, the scale folded with log2 e) and its row reductions (two shuffles
// across the lane groups) run on the lane's own row, and the probabilities
// are already the B operand of O^T = V^T P^T, whose D layout again gives a
// lane four dimensions of its row to rescale. V^T is staged in LDS with the
// keys of each 32-key slice in the order that layout implies: within a slice,
// operand position 8 g + i holds key 4 g + i for i < 4 and 16 + 4 g + i - 4
// otherwise. Operands are split into bf16 hi + lo terms as in
// attn_bf16_kernel (q and p always; an f32 cache's keys and values too).
template <typename KV>
struct GqaShape;
template <>
struct GqaShape<uint16_t> {
    static constexpr int NW = 8;
};
template <>
struct GqaShape<float> {
    static constexpr int NW = 8;
};

template <typename KV>
__global__ __launch_bounds__(64 * GqaShape<KV>::NW, 8 / GqaShape<KV>::NW) void attn_gqa_kernel(int gxy, int n, int gnh, const float *__restrict__ q, AttnKernelArgs a) {
    constexpr bool F32 = sizeof(KV) == 4;
    constexpr int NW = GqaShape<KV>::NW, NT = 64 * NW, SETS = kGqaRows / 16 / NW, RW = 16 * SETS;
    constexpr int HD = 128, KT = kGqaKeys;
    constexpr int KSB = HD + 8;  // K row stride (bf16): 16 rows of a fragment read land on 16 bank groups
    constexpr int VTS = KT + 8;  // V^T row stride (bf16), likewise
    constexpr int KU = KT * (HD / 8) / NT;  // K units (key, 8 dims) a thread stages
    constexpr int VU = 64 * (KT / 8) / NT;  // V items (dimension pair, operand group) a thread stages
    constexpr float kLog2e = 1.4426950408889634f, kLn2 = 0.6931471805599453f;
    __shared__ uint4 ksh[KT * KSB / 8], ksl[F32 ? KT * KSB / 8 : 1];
    __shared__ uint4 vth[HD * VTS / 8], vtl[F32 ? HD * VTS / 8 : 1];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    // Leading arguments, preloaded: the grid's x | y << 16, the query rows,
    // the group | q heads << 16 and q (a's own fields).
    const int G = gnh & 0xffff, QT = kGqaRows / G;
    // Blocks in order of decreasing work (the last token tiles, which see
    // the most keys, first), as in attn_planes_kernel.
    const int gx = gxy & 0xffff, gy = gxy >> 16, lin = (int)blockIdx.x + (int)blockIdx.y * gx;
    const int g = lin % gy;
    const int t0 = (gx - 1 - lin / gy) * QT;
    const int nq = n - t0 < QT ? n - t0 : QT;
    const long long pos = a.pos_dev ? *a.pos_dev : a.pos;
    // Rows of set s: block row r = RW wave + 16 s + li is head g G + r / QT,
    // token t0 + r % QT.
    int qloc[SETS], head[SETS];
    uint4 qh[SETS][HD / 32], ql[SETS][HD / 32];
#pragma unroll
    for (int s = 0; s < SETS; ++s) {
        const int r = RW * wave + 16 * s + li;
        qloc[s] = r % QT;
        head[s] = g * G + r / QT;
        const float *qp = q + ((long long)(t0 + (qloc[s] < nq ? qloc[s] : 0)) * (gnh >> 16) + head[s]) * HD + 8 * lg;
#pragma unroll
        for (int c = 0; c < HD / 32; ++c) {
            float f[8];
            const float4 x0 = *reinterpret_cast<const float4 *>(qp + 32 * c);
            const float4 x1 = *reinterpret_cast<const float4 *>(qp + 32 * c + 4);
            f[0] = x0.x; f[1] = x0.y; f[2] = x0.z; f[3] = x0.w;
            f[4] = x1.x; f[5] = x1.y; f[6] = x1.z; f[7] = x1.w;
            if (qloc[s] >= nq)
#pragma unroll
                for (int e = 0; e < 8; ++e) f[e] = 0.f;
            split8(f, qh[s][c], ql[s][c]);
        }
    }
    const KV *kb = reinterpret_cast<const KV *>(a.k) + (long long)g * a.head_stride;
    const KV *vb = reinterpret_cast<const KV *>(a.v) + (long long)g * a.head_stride;
    const long long last = pos + t0 + nq - 1;  // the block's last query position
    // This wave's last query position (rows past n excluded).
    const int wq = QT >= RW ? (RW * wave) % QT + RW - 1 : QT - 1;
    const long long wlast = pos + t0 + (wq < nq - 1 ? wq : nq - 1);
    const long long ntiles = last / KT + 1, z = blockIdx.z;
    const long long kt0 = z * ntiles / a.nsplit, kt1 = (z + 1) * ntiles / a.nsplit;
    floatx4 o[SETS][HD / 16];
    float m[SETS], l[SETS];
#pragma unroll
    for (int s = 0; s < SETS; ++s) {
        m[s] = -INFINITY;
        l[s] = 0.f;
#pragma unroll
        for (int d = 0; d < HD / 16; ++d) o[s][d] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    const float scale2 = a.scale * kLog2e;
    // Staging. K unit u = tid + NT i is key u / 16, dims 8 (u % 16) + [0, 8).
    // V item u = tid + NT i is dimensions 2 (u % 64) + {0, 1} of operand group
    // u / 64 (slice (u / 64) / 4, group (u / 64) % 4). Positions past the
    // block's last query read as 0. A bf16 cache stays packed in registers
    // (its lo terms are 0); an f32 cache is held as f32 and split when stored.
    const int vd = 2 * (tid & 63);
    auto kkey = [&](int i) { return (tid + NT * i) >> 4; };
    auto kch = [&](int i) { return (tid + NT * i) & 15; };
    auto vgrp = [&](int i) { return (tid + NT * i) >> 6; };
    auto vkey = [&](int i, int j) {  // key (within the tile) at operand position j of item i
        const int gr = vgrp(i), sigma = gr >> 2, gp = gr & 3;
        return 32 * sigma + (j < 4 ? 4 * gp + j : 16 + 4 * gp + j - 4);
    };
    uint4 kpk[F32 ? 1 : KU];
    uint32_t vpk[F32 ? 1 : VU][8];
    float4 kf[F32 ? KU : 1][2];
    float2 vf[F32 ? VU : 1][8];
    auto fetch = [&](long long c0) {
#pragma unroll
        for (int i = 0; i < KU; ++i) {
            const long long pk = c0 + kkey(i);
            const KV *src = kb + pk * a.pos_stride + 8 * kch(i);
            if constexpr (F32) {
                kf[i][0] = pk <= last ? *reinterpret_cast<const float4 *>(src) : make_float4(0.f, 0.f, 0.f, 0.f);
                kf[i][1] = pk <= last ? *reinterpret_cast<const float4 *>(src + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
                kpk[i] = pk <= last ? *reinterpret_cast<const uint4 *>(src) : make_uint4(0, 0, 0, 0);
            }
        }
#pragma unroll
        for (int i = 0; i < VU; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const long long pv = c0 + vkey(i, j);
                const KV *src = vb + pv * a.pos_stride + vd;
                if constexpr (F32)
                    vf[i][j] = pv <= last ? *reinterpret_cast<const float2 *>(src) : make_float2(0.f, 0.f);
                else
                    vpk[i][j] = pv <= last ? *reinterpret_cast<const uint32_t *>(src) : 0u;
            }
    };
    const long long cend = kt1 * KT;
    if (kt0 < kt1) fetch(kt0 * KT);
    for (long long c0 = kt0 * KT; c0 < cend; c0 += KT) {
        __syncthreads();  // the previous tile is consumed
#pragma unroll
        for (int i = 0; i < KU; ++i) {
            const int off = (kkey(i) * KSB + 8 * kch(i)) / 8;
            if constexpr (F32) {
                const float f[8] = {kf[i][0].x, kf[i][0].y, kf[i][0].z, kf[i][0].w,
                                    kf[i][1].x, kf[i][1].y, kf[i][1].z, kf[i][1].w};
                split8(f, ksh[off], ksl[off]);
            } else {
                ksh[off] = kpk[i];
            }
        }
#pragma unroll
        for (int i = 0; i < VU; ++i) {
            const int gr = vgrp(i);
            const int off0 = (vd * VTS + 32 * (gr >> 2) + 8 * (gr & 3)) / 8, off1 = off0 + VTS / 8;
            if constexpr (F32) {
                float f0[8], f1[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    f0[j] = vf[i][j].x;
                    f1[j] = vf[i][j].y;
                }
                split8(f0, vth[off0], vtl[off0]);
                split8(f1, vth[off1], vtl[off1]);
            } else {
                uint32_t e[4], d[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t w0 = vpk[i][2 * j], w1 = vpk[i][2 * j + 1];
                    e[j] = (w0 & 0xFFFFu) | (w1 << 16);          // dimension vd
                    d[j] = (w0 >> 16) | (w1 & 0xFFFF0000u);      // dimension vd + 1
                }
                vth[off0] = make_uint4(e[0], e[1], e[2], e[3]);
                vth[off1] = make_uint4(d[0], d[1], d[2], d[3]);
            }
        }
        __syncthreads();
        if (c0 + KT < cend) fetch(c0 + KT);
        if (c0 > wlast) continue;  // every query of this wave precedes the tile
        // S^T: keys c0 + 16 j + [0, 16) down, the set's 16 rows across.
        floatx4 st[SETS][KT / 16];
#pragma unroll
        for (int s = 0; s < SETS; ++s)
#pragma unroll
            for (int j = 0; j < KT / 16; ++j) st[s][j] = floatx4{0.f, 0.f, 0.f, 0.f};
        // Per 32-dimension step: the tile's four key fragments first (one
        // base address, constant offsets), then each product term across the
        // four independent accumulators, so that no MFMA waits on the one
        // before it. Each accumulator still adds hi*hi, hi*lo, lo*hi in turn.
        const uint4 *kbh = ksh + (li * KSB + 8 * lg) / 8;
        const uint4 *kbl = ksl + (F32 ? (li * KSB + 8 * lg) / 8 : 0);
#pragma unroll
        for (int c = 0; c < HD / 32; ++c) {
            bf16x8_t kh[KT / 16], kl[F32 ? KT / 16 : 1];
#pragma unroll
            for (int j = 0; j < KT / 16; ++j) kh[j] = as_bf8(kbh[(16 * j * KSB + 32 * c) / 8]);
            if constexpr (F32)
#pragma unroll
                for (int j = 0; j < KT / 16; ++j) kl[j] = as_bf8(kbl[(16 * j * KSB + 32 * c) / 8]);
#pragma unroll
            for (int s = 0; s < SETS; ++s)
#pragma unroll
                for (int j = 0; j < KT / 16; ++j)
                    st[s][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh[j], as_bf8(qh[s][c]), st[s][j], 0, 0, 0);
#pragma unroll
            for (int s = 0; s < SETS; ++s)
#pragma unroll
                for (int j = 0; j < KT / 16; ++j)
                    st[s][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh[j], as_bf8(ql[s][c]), st[s][j], 0, 0, 0);
            if constexpr (F32)
#pragma unroll
                for (int s = 0; s < SETS; ++s)
#pragma unroll
                    for (int j = 0; j < KT / 16; ++j)
                        st[s][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl[j], as_bf8(qh[s][c]), st[s][j], 0, 0, 0);
        }
        // Causal mask and online softmax of the lane's row; p overwrites st.
#pragma unroll
        for (int s = 0; s < SETS; ++s) {
            // Key c0 + 16 j + 4 lg + e is visible to the row when 16 j + e <=
            // lim (32-bit: the tile holds 64 keys); a row past n sees none.
            const long long qpos = pos + t0 + qloc[s];
            const long long d = qpos - c0 - 4 * lg;
            const int lim = qloc[s] >= nq ? -1 : d > KT ? KT : (int)d;
            float mx = -INFINITY;
#pragma unroll
            for (int j = 0; j < KT / 16; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float v = 16 * j + e <= lim ? st[s][j][e] * scale2 : -INFINITY;
                    st[s][j][e] = v;
                    mx = fmaxf(mx, v);
                }
            mx = rows_max(mx);
            const float mn = fmaxf(m[s], mx);
            const float alpha = m[s] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[s] - mn);
            float sum = 0.f;
#pragma unroll
            for (int j = 0; j < KT / 16; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float v = st[s][j][e];
                    const float p = v == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(v - mn);
                    st[s][j][e] = p;
                    sum += p;
                }
            sum = rows_sum(sum);
            l[s] = l[s] * alpha + sum;
            m[s] = mn;
#pragma unroll
            for (int d = 0; d < HD / 16; ++d)
#pragma unroll
                for (int e = 0; e < 4; ++e) o[s][d][e] *= alpha;
        }
        // O^T += V^T P^T over the tile's two 32-key slices.
#pragma unroll
        for (int sg = 0; sg < KT / 32; ++sg) {
            uint4 ph[SETS], pl[SETS];
#pragma unroll
            for (int s = 0; s < SETS; ++s) {
                const float f[8] = {st[s][2 * sg][0],     st[s][2 * sg][1],     st[s][2 * sg][2],
                                    st[s][2 * sg][3],     st[s][2 * sg + 1][0], st[s][2 * sg + 1][1],
                                    st[s][2 * sg + 1][2], st[s][2 * sg + 1][3]};
                split8(f, ph[s], pl[s]);
            }
            // Four dimension tiles at a time: their V^T fragments first, then
            // each product term across the four accumulators.
            const uint4 *vbh = vth + (li * VTS + 32 * sg + 8 * lg) / 8;
            const uint4 *vbl = vtl + (F32 ? (li * VTS + 32 * sg + 8 * lg) / 8 : 0);
#pragma unroll
            for (int d0 = 0; d0 < HD / 16; d0 += 4) {
                bf16x8_t vh[4], vl[F32 ? 4 : 1];
#pragma unroll
                for (int i = 0; i < 4; ++i) vh[i] = as_bf8(vbh[(16 * (d0 + i) * VTS) / 8]);
                if constexpr (F32)
#pragma unroll
                    for (int i = 0; i < 4; ++i) vl[i] = as_bf8(vbl[(16 * (d0 + i) * VTS) / 8]);
#pragma unroll
                for (int s = 0; s < SETS; ++s)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        o[s][d0 + i] =
                            __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh[i], as_bf8(ph[s]), o[s][d0 + i], 0, 0, 0);
#pragma unroll
                for (int s = 0; s < SETS; ++s)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        o[s][d0 + i] =
                            __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh[i], as_bf8(pl[s]), o[s][d0 + i], 0, 0, 0);
                if constexpr (F32)
#pragma unroll
                    for (int s = 0; s < SETS; ++s)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            o[s][d0 + i] =
                                __builtin_amdgcn_mfma_f32_16x16x32_bf16(vl[i], as_bf8(ph[s]), o[s][d0 + i], 0, 0, 0);
            }
        }
    }
    // o[s][d][e] is dimension 16 d + 4 lg + e of the lane's row.
#pragma unroll
    for (int s = 0; s < SETS; ++s) {
        if (qloc[s] >= nq) continue;
        const long long th = (long long)(t0 + qloc[s]) * a.n_heads + head[s];
        if (a.nsplit == 1) {
            const float inv = 1.f / l[s];
#pragma unroll
            for (int d = 0; d < HD / 16; ++d) {
                const float4 v = make_float4(o[s][d][0] * inv, o[s][d][1] * inv, o[s][d][2] * inv, o[s][d][3] * inv);
                const long long off = th * HD + 16 * d + 4 * lg;
                if (a.out_hi) {
                    uint2 h, w;
                    split_bf16x4(v, h, w);
                    *reinterpret_cast<uint2 *>(a.out_hi + off) = h;
                    *reinterpret_cast<uint2 *>(a.out_lo + off) = w;
                } else {
                    *reinterpret_cast<float4 *>(a.out + off) = v;
                }
            }
        } else {
            const long long slot = th * a.nsplit + z;
#pragma unroll
            for (int d = 0; d < HD / 16; ++d)
                *reinterpret_cast<float4 *>(a.part_acc + slot * HD + 16 * d + 4 * lg) =
                    make_float4(o[s][d][0], o[s][d][1], o[s][d][2], o[s][d][3]);
            if (lg == 0) {
                a.part_ml[slot * 2] = m[s] * kLn2;
                a.part_ml[slot * 2 + 1] = l[s];
            }
        }
    }
}

// ---- prefill attention over bf16 planes of an f32 cache ----
//
// attn_gqa_kernel splits every f32 key and value into bf16 hi + lo in every
// block that reads it: with a 2048-token chunk, each 64-key tile is split by
// every token tile of its KV group, in VALU and registers, between two block
// barriers per tile. Here a first kernel writes the split once per layer into
// four bf16 planes: K hi / lo row-major [kv head][position][128], V^T hi / lo
// dimension-major [kv head][128][position] with each 32-key slice's columns
// in the P^T operand order of attn_gqa_kernel (column 8 g + i holds key
// 4 g + i for i < 4 and 16 + 4 g + i - 4 otherwise). The attention blocks
// then stage tiles with direct global -> LDS loads into a two-stage ring, one
// block barrier per tile, the next tile in flight during this one's
// products. The planes carry the same bf16 terms and the products run in the
// same order, so the result is attn_gqa_kernel's, bit for bit.

struct KvPlaneArgs {
    const float *k, *v;           // the layer's caches: head g, position p at g head_stride + p pos_stride
    long long head_stride, pos_stride;
    uint16_t *kh, *kl, *vh, *vl;  // the planes, each n_kv_heads x 128 x plane_len bf16
    long long plane_len;          // positions a plane holds per head (a multiple of 64)
    long long valid;              // positions [0, valid) hold keys; later ones of a tile become zeros
};

// One block per (64-position tile, KV head).
__global__ __launch_bounds__(256) void kv_planes_kernel(KvPlaneArgs a) {
    constexpr int HD = 128;
    __shared__ float vs[64][HD + 1];
    const int g = blockIdx.y, tid = threadIdx.x;
    const long long p0 = (long long)blockIdx.x * 64;
    const float *kb = a.k + (long long)g * a.head_stride, *vb = a.v + (long long)g * a.head_stride;
    // Keys: 64 rows x 16 chunks of 8 dimensions.
    for (int u = tid; u < 64 * 16; u += 256) {
        const int r = u >> 4, ch = u & 15;
        const long long p = p0 + r;
        float f[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        if (p < a.valid) {
            const float4 x0 = *reinterpret_cast<const float4 *>(kb + p * a.pos_stride + 8 * ch);
            const float4 x1 = *reinterpret_cast<const float4 *>(kb + p * a.pos_stride + 8 * ch + 4);
            f[0] = x0.x; f[1] = x0.y; f[2] = x0.z; f[3] = x0.w;
            f[4] = x1.x; f[5] = x1.y; f[6] = x1.z; f[7] = x1.w;
        }
        uint4 h, l;
        split8(f, h, l);
        const long long o = ((long long)g * a.plane_len + p) * HD + 8 * ch;
        *reinterpret_cast<uint4 *>(a.kh + o) = h;
        *reinterpret_cast<uint4 *>(a.kl + o) = l;
    }
    // Values: the tile through LDS, then 128 dimensions x 8 column chunks.
    for (int u = tid; u < 64 * (HD / 4); u += 256) {
        const int r = u / (HD / 4), c4 = u % (HD / 4);
        const long long p = p0 + r;
        const float4 x =
            p < a.valid ? *reinterpret_cast<const float4 *>(vb + p * a.pos_stride + 4 * c4) : make_float4(0.f, 0.f, 0.f, 0.f);
        vs[r][4 * c4] = x.x;
        vs[r][4 * c4 + 1] = x.y;
        vs[r][4 * c4 + 2] = x.z;
        vs[r][4 * c4 + 3] = x.w;
    }
    __syncthreads();
    for (int u = tid; u < HD * 8; u += 256) {
        const int d = u >> 3, pc = u & 7, slice = pc >> 2, grp = pc & 3;
        float f[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) f[i] = vs[32 * slice + (i < 4 ? 4 * grp + i : 16 + 4 * grp + i - 4)][d];
        uint4 h, l;
        split8(f, h, l);
        const long long o = ((long long)g * HD + d) * a.plane_len + p0 + 8 * pc;
        *reinterpret_cast<uint4 *>(a.vh + o) = h;
        *reinterpret_cast<uint4 *>(a.vl + o) = l;
    }
}

// Waves of an attn_planes_kernel block (each ROWS / 16 / kPlaneWaves sets of
// 16 (token, head) rows). Two sets a wave halve the LDS reads per product
// (every wave reads the whole tile) and double the products per staged
// tile, at 246 VGPRs, still two waves a SIMD: 4B-shape 8192-token prefill
// 175.9 -> 168.1 ms, Qwen3-0.6B 8192 tokens 39.7 -> 36.6 ms. With half the
// blocks they are slower where blocks are few (0.6B, 512 tokens: 3.05 ->
// 3.22 ms), so they run only once the launch has a block per CU unsplit.
constexpr int kPlaneWaves = 8, kPlaneRowsWide = 256;

static bool plane_rows_wide(size_t n, int group, int n_kv_heads) {
    const size_t qt = (size_t)(kPlaneRowsWide / group);
    return (n + qt - 1) / qt * (size_t)n_kv_heads >= 256;
}

struct PlaneRefs {
    const uint16_t *kh, *kl, *vh, *vl;
    long long plane_len;
};

// attn_gqa_kernel<float> with its tiles staged from the planes. LDS: two
// stages of four 16 KB tiles (K hi, K lo: 64 keys x 256 B; V^T hi, V^T lo:
// 128 dimensions x 128 B), rows XOR-swizzled in 16-byte chunks so that a
// fragment read's 16 rows land on distinct banks: K row r keeps logical
// chunk c at c ^ (r & 15), V^T row r at c ^ ((r >> 1) & 7) (two 128-byte
// rows share a bank line).
template <int NW, int ROWS>
__global__ __launch_bounds__(64 * NW, 1) void attn_planes_kernel(int gxy, int n, int gnh, const float *__restrict__ q,
                                                                 AttnKernelArgs a, PlaneRefs pl) {
    constexpr int SETS = ROWS / 16 / NW, RW = 16 * SETS;
    constexpr int SPW = 16 / NW;  // 1 KB spans a wave fills of each 16 KB tile
    constexpr int HD = 128, KT = kGqaKeys;
    static_assert(KT == 64 && SETS >= 1, "64-key tiles");
    constexpr float kLog2e = 1.4426950408889634f, kLn2 = 0.6931471805599453f;
    struct alignas(16) Stage {
        uint4 kh[KT * 16], kl[KT * 16];  // [key][16 chunks]
        uint4 vh[HD * 8], vl[HD * 8];    // [dimension][8 chunks]
    };
    __shared__ Stage ring[2];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lg = lane >> 4;
    // Leading arguments as attn_gqa_kernel's.
    const int G = gnh & 0xffff, QT = ROWS / G;
    // Blocks in order of decreasing work: a token tile attends to every key
    // up to its last query, so the last tiles have the most; launching them
    // first (every KV group's last tile, then the one before, ...) keeps the
    // lightest blocks for the end of the launch instead of the heaviest.
    const int gx = gxy & 0xffff, gy = gxy >> 16, lin = (int)blockIdx.x + (int)blockIdx.y * gx;
    const int g = lin % gy;
    const int t0 = (gx - 1 - lin / gy) * QT;
    const int nq = n - t0 < QT ? n - t0 : QT;
    const long long pos = a.pos;
    int qloc[SETS], head[SETS];
    uint4 qh[SETS][HD / 32], ql[SETS][HD / 32];
#pragma unroll
    for (int s = 0; s < SETS; ++s) {
        const int r = RW * wave + 16 * s + li;
        qloc[s] = r % QT;
        head[s] = g * G + r / QT;
        const float *qp = q + ((long long)(t0 + (qloc[s] < nq ? qloc[s] : 0)) * (gnh >> 16) + head[s]) * HD + 8 * lg;
#pragma unroll
        for (int c = 0; c < HD / 32; ++c) {
            float f[8];
            const float4 x0 = *reinterpret_cast<const float4 *>(qp + 32 * c);
            const float4 x1 = *reinterpret_cast<const float4 *>(qp + 32 * c + 4);
            f[0] = x0.x; f[1] = x0.y; f[2] = x0.z; f[3] = x0.w;
            f[4] = x1.x; f[5] = x1.y; f[6] = x1.z; f[7] = x1.w;
            if (qloc[s] >= nq)
#pragma unroll
                for (int e = 0; e < 8; ++e) f[e] = 0.f;
            split8(f, qh[s][c], ql[s][c]);
        }
    }
    const long long last = pos + t0 + nq - 1;
    const int wq = QT >= RW ? (RW * wave) % QT + RW - 1 : QT - 1;
    const long long wlast = pos + t0 + (wq < nq - 1 ? wq : nq - 1);
    const long long ntiles = last / KT + 1, z = blockIdx.z;
    const long long kt0 = z * ntiles / a.nsplit, kt1 = (z + 1) * ntiles / a.nsplit;
    floatx4 o[SETS][HD / 16];
    float m[SETS], l[SETS];
#pragma unroll
    for (int s = 0; s < SETS; ++s) {
        m[s] = -INFINITY;
        l[s] = 0.f;
#pragma unroll
        for (int d = 0; d < HD / 16; ++d) o[s][d] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    const float scale2 = a.scale * kLog2e;
    const uint16_t *khg = pl.kh + (long long)g * pl.plane_len * HD, *klg = pl.kl + (long long)g * pl.plane_len * HD;
    const uint16_t *vhg = pl.vh + (long long)g * HD * pl.plane_len, *vlg = pl.vl + (long long)g * HD * pl.plane_len;
    // Each wave fills SPW 1 KB spans of each tile: K spans are 4 keys, V^T
    // spans 8 dimensions.
    auto issue = [&](Stage &st, long long c0) {
#pragma unroll
        for (int i = 0; i < SPW; ++i) {
            const int span = SPW * wave + i, p = span * 64 + lane, row = p >> 4, pc = p & 15;
            const long long off = (c0 + row) * HD + 8 * (pc ^ (row & 15));
            dma16(khg + off, st.kh + span * 64);
            dma16(klg + off, st.kl + span * 64);
        }
#pragma unroll
        for (int i = 0; i < SPW; ++i) {
            const int span = SPW * wave + i, p = span * 64 + lane, row = p >> 3, pc = p & 7;
            const long long off = (long long)row * pl.plane_len + c0 + 8 * (pc ^ ((row >> 1) & 7));
            dma16(vhg + off, st.vh + span * 64);
            dma16(vlg + off, st.vl + span * 64);
        }
    };
    const long long cend = kt1 * KT;
    if (kt0 < kt1) issue(ring[0], kt0 * KT);
    int sn = 0;
    for (long long c0 = kt0 * KT; c0 < cend; c0 += KT, sn ^= 1) {
        // This wave's loads of the tile are done; the barrier makes every
        // wave's visible and frees the other stage (read during the last tile).
        wait_vm<0>();
        __syncthreads();
        if (c0 + KT < cend) issue(ring[sn ^ 1], c0 + KT);
        if (c0 > wlast) continue;  // every query of this wave precedes the tile
        const Stage &st = ring[sn];
        floatx4 sc[SETS][KT / 16];
#pragma unroll
        for (int s = 0; s < SETS; ++s)
#pragma unroll
            for (int j = 0; j < KT / 16; ++j) sc[s][j] = floatx4{0.f, 0.f, 0.f, 0.f};
        // S^T = K Q^T: key rows 16 j + li, logical chunk 4 c + lg.
#pragma unroll
        for (int c = 0; c < HD / 32; ++c) {
            const int pcv = (4 * c + lg) ^ li;
            bf16x8_t kh[KT / 16], kl[KT / 16];
#pragma unroll
            for (int j = 0; j < KT / 16; ++j) kh[j] = as_bf8(st.kh[(16 * j + li) * 16 + pcv]);
#pragma unroll
            for (int j = 0; j < KT / 16; ++j) kl[j] = as_bf8(st.kl[(16 * j + li) * 16 + pcv]);
#pragma unroll
            for (int s = 0; s < SETS; ++s)
#pragma unroll
                for (int j = 0; j < KT / 16; ++j)
                    sc[s][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh[j], as_bf8(qh[s][c]), sc[s][j], 0, 0, 0);
#pragma unroll
            for (int s = 0; s < SETS; ++s)
#pragma unroll
                for (int j = 0; j < KT / 16; ++j)
                    sc[s][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh[j], as_bf8(ql[s][c]), sc[s][j], 0, 0, 0);
#pragma unroll
            for (int s = 0; s < SETS; ++s)
#pragma unroll
                for (int j = 0; j < KT / 16; ++j)
                    sc[s][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl[j], as_bf8(qh[s][c]), sc[s][j], 0, 0, 0);
        }
#pragma unroll
        for (int s = 0; s < SETS; ++s) {
            const long long qpos = pos + t0 + qloc[s];
            const long long d = qpos - c0 - 4 * lg;
            const int lim = qloc[s] >= nq ? -1 : d > KT ? KT : (int)d;
            float mx = -INFINITY;
#pragma unroll
            for (int j = 0; j < KT / 16; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float v = 16 * j + e <= lim ? sc[s][j][e] * scale2 : -INFINITY;
                    sc[s][j][e] = v;
                    mx = fmaxf(mx, v);
                }
            mx = rows_max(mx);
            const float mn = fmaxf(m[s], mx);
            const float alpha = m[s] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[s] - mn);
            float sum = 0.f;
#pragma unroll
            for (int j = 0; j < KT / 16; ++j)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float v = sc[s][j][e];
                    const float p = v == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(v - mn);
                    sc[s][j][e] = p;
                    sum += p;
                }
            sum = rows_sum(sum);
            l[s] = l[s] * alpha + sum;
            m[s] = mn;
            // No row of the wave raised its maximum: alpha is exactly 1 and
            // the rescale changes nothing (4B 8192-token prefill 153.6-154.6
            // -> 152.8-153.3 ms in three paired runs).
            if (__builtin_amdgcn_ballot_w64(alpha != 1.f) != 0) {
#pragma unroll
                for (int d2 = 0; d2 < HD / 16; ++d2)
#pragma unroll
                    for (int e = 0; e < 4; ++e) o[s][d2][e] *= alpha;
            }
        }
        // O^T += V^T P^T: dimension rows 16 (d0 + i) + li, logical chunk 4 sg + lg.
#pragma unroll
        for (int sg = 0; sg < KT / 32; ++sg) {
            uint4 ph[SETS], pq[SETS];
#pragma unroll
            for (int s = 0; s < SETS; ++s) {
                const float f[8] = {sc[s][2 * sg][0],     sc[s][2 * sg][1],     sc[s][2 * sg][2],
                                    sc[s][2 * sg][3],     sc[s][2 * sg + 1][0], sc[s][2 * sg + 1][1],
                                    sc[s][2 * sg + 1][2], sc[s][2 * sg + 1][3]};
                split8(f, ph[s], pq[s]);
            }
            const int pcv = (4 * sg + lg) ^ ((li >> 1) & 7);
#pragma unroll
            for (int d0 = 0; d0 < HD / 16; d0 += 4) {
                bf16x8_t vh[4], vl[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) vh[i] = as_bf8(st.vh[(16 * (d0 + i) + li) * 8 + pcv]);
#pragma unroll
                for (int i = 0; i < 4; ++i) vl[i] = as_bf8(st.vl[(16 * (d0 + i) + li) * 8 + pcv]);
#pragma unroll
                for (int s = 0; s < SETS; ++s)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        o[s][d0 + i] =
                            __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh[i], as_bf8(ph[s]), o[s][d0 + i], 0, 0, 0);
#pragma unroll
                for (int s = 0; s < SETS; ++s)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        o[s][d0 + i] =
                            __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh[i], as_bf8(pq[s]), o[s][d0 + i], 0, 0, 0);
#pragma unroll
                for (int s = 0; s < SETS; ++s)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        o[s][d0 + i] =
                            __builtin_amdgcn_mfma_f32_16x16x32_bf16(vl[i], as_bf8(ph[s]), o[s][d0 + i], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int s = 0; s < SETS; ++s) {
        if (qloc[s] >= nq) continue;
        const long long th = (long long)(t0 + qloc[s]) * a.n_heads + head[s];
        if (a.nsplit == 1) {
            const float inv = 1.f / l[s];
#pragma unroll
            for (int d = 0; d < HD / 16; ++d) {
                const float4 v = make_float4(o[s][d][0] * inv, o[s][d][1] * inv, o[s][d][2] * inv, o[s][d][3] * inv);
                const long long off = th * HD + 16 * d + 4 * lg;
                if (a.out_hi) {
                    uint2 h, w;
                    split_bf16x4(v, h, w);
                    *reinterpret_cast<uint2 *>(a.out_hi + off) = h;
                    *reinterpret_cast<uint2 *>(a.out_lo + off) = w;
                } else {
                    *reinterpret_cast<float4 *>(a.out + off) = v;
                }
            }
        } else {
            const long long slot = th * a.nsplit + z;
#pragma unroll
            for (int d = 0; d < HD / 16; ++d)
                *reinterpret_cast<float4 *>(a.part_acc + slot * HD + 16 * d + 4 * lg) =
                    make_float4(o[s][d][0], o[s][d][1], o[s][d][2], o[s][d][3]);
            if (lg == 0) {
                a.part_ml[slot * 2] = m[s] * kLn2;
                a.part_ml[slot * 2 + 1] = l[s];
            }
        }
    }
}

template <int HD>
static hipError_t attn_launch(hipStream_t s, AttnKernelArgs k, size_t n) {
    dim3 grid((unsigned)(n * (size_t)k.n_kv_heads * (size_t)k.nsplit));
    if (HD == 128 && k.group >= 1 && k.group <= kAttnMaxGroup) {
        if (k.kv_bf16)
            attn_rows_kernel<uint16_t><<<grid, 256, 0, s>>>(k);
        else
            attn_rows_kernel<float><<<grid, 256, 0, s>>>(k);
    } else if (k.kv_bf16)
        attn_split_kernel<HD, uint16_t><<<grid, 256, 0, s>>>(k);
    else
        attn_split_kernel<HD, float><<<grid, 256, 0, s>>>(k);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && k.nsplit > 1)
        e = launch_attn_combine(s, k.out, k.part_acc, k.part_ml, n * (size_t)k.n_heads, k.nsplit, HD);
    if (e != hipSuccess || !k.out_hi) return e;
    return launch_gemm_split(s, k.out, n, (size_t)k.n_heads * HD, k.out_hi, k.out_lo);
}

hipError_t launch_attention(hipStream_t s, const AttnKernelArgs &k, size_t n, size_t head_dim) {
    if (n == 0) return hipSuccess;
    if (head_dim == 128 && n >= kAttnTileMin) {
        if (k.group >= 1 && k.group <= 8 && 8 % k.group == 0 && k.n_kv_heads * k.group == k.n_heads) {
            const int qt = kGqaRows / k.group;
            dim3 grid((unsigned)((n + qt - 1) / qt), (unsigned)k.n_kv_heads, (unsigned)k.nsplit);
            if (grid.x > 0xffff || grid.y > 0xffff || k.n_heads > 0x7fff) return hipErrorInvalidValue;
            const int gxy = (int)(grid.x | grid.y << 16), gnh = k.group | k.n_heads << 16;
            if (k.kv_bf16)
                attn_gqa_kernel<uint16_t><<<grid, 64 * GqaShape<uint16_t>::NW, 0, s>>>(gxy, (int)n, gnh, k.q, k);
            else
                attn_gqa_kernel<float><<<grid, 64 * GqaShape<float>::NW, 0, s>>>(gxy, (int)n, gnh, k.q, k);
        } else {
            dim3 grid((unsigned)((n + kMQT - 1) / kMQT), (unsigned)k.n_heads, (unsigned)k.nsplit);
            if (k.kv_bf16)
                attn_bf16_kernel<uint16_t><<<grid, 256, 0, s>>>(k, (int)n);
            else
                attn_bf16_kernel<float><<<grid, 256, 0, s>>>(k, (int)n);
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess || k.nsplit == 1) return e;
        return launch_attn_combine(s, k.out, k.part_acc, k.part_ml, n * (size_t)k.n_heads, k.nsplit, 128, k.out_hi,
                                   k.out_lo);
    }
    switch (head_dim) {
    case 64: return attn_launch<64>(s, k, n);
    case 128: return attn_launch<128>(s, k, n);
    case 256: return attn_launch<256>(s, k, n);
    default: return hipErrorInvalidValue;
    }
}

size_t attention_planes_bytes(size_t max_len, size_t n_kv_heads) {
    return 4 * n_kv_heads * 128 * ((max_len + 63) / 64 * 64) * sizeof(uint16_t);
}

bool attention_planes_supported(const AttnKernelArgs &k, size_t n, size_t head_dim) {
    return head_dim == 128 && n >= kAttnTileMin && !k.kv_bf16 && !k.pos_dev && k.group >= 1 && k.group <= 8 &&
           8 % k.group == 0 && k.n_kv_heads * k.group == k.n_heads && k.pos_stride % 4 == 0 &&
           k.head_stride % 4 == 0;
}

PlanePtrs attention_planes_of(void *planes, size_t max_len, size_t n_kv_heads) {
    const long long plane_len = (long long)((max_len + 63) / 64 * 64);
    const size_t plane = n_kv_heads * 128 * (size_t)plane_len;
    uint16_t *p0 = static_cast<uint16_t *>(planes);
    return PlanePtrs{p0, p0 + plane, p0 + 2 * plane, p0 + 3 * plane, plane_len};
}

hipError_t launch_kv_planes(hipStream_t s, const AttnKernelArgs &k, size_t valid, void *planes, size_t planes_bytes,
                            size_t max_len) {
    if (valid == 0) return hipSuccess;
    if (!planes || valid > max_len || k.kv_bf16 || k.pos_stride % 4 || k.head_stride % 4 ||
        attention_planes_bytes(max_len, (size_t)k.n_kv_heads) > planes_bytes || (uintptr_t)planes % 16)
        return hipErrorInvalidValue;
    const PlanePtrs pp = attention_planes_of(planes, max_len, (size_t)k.n_kv_heads);
    KvPlaneArgs c{};
    c.k = static_cast<const float *>(k.k);
    c.v = static_cast<const float *>(k.v);
    c.head_stride = k.head_stride;
    c.pos_stride = k.pos_stride;
    c.kh = pp.kh;
    c.kl = pp.kl;
    c.vh = pp.vh;
    c.vl = pp.vl;
    c.plane_len = pp.plane_len;
    c.valid = (long long)valid;
    kv_planes_kernel<<<dim3((unsigned)((c.valid + 63) / 64), (unsigned)k.n_kv_heads), 256, 0, s>>>(c);
    return hipGetLastError();
}

hipError_t launch_attention_planes(hipStream_t s, const AttnKernelArgs &k, size_t n, size_t head_dim, void *planes,
                                   size_t planes_bytes, size_t max_len, bool split_kv) {
    if (n == 0) return hipSuccess;
    if (!attention_planes_supported(k, n, head_dim) || !planes || k.pos < 0 || (size_t)k.pos + n > max_len ||
        attention_planes_bytes(max_len, (size_t)k.n_kv_heads) > planes_bytes || (uintptr_t)planes % 16)
        return hipErrorInvalidValue;
    hipError_t e;
    if (split_kv) {
        e = launch_kv_planes(s, k, (size_t)k.pos + n, planes, planes_bytes, max_len);
        if (e != hipSuccess) return e;
    }
    const PlanePtrs pp = attention_planes_of(planes, max_len, (size_t)k.n_kv_heads);
    const long long plane_len = pp.plane_len;
    const PlaneRefs pr{pp.kh, pp.kl, pp.vh, pp.vl, plane_len};
    // Rows a block: the wide form only unsplit, so that every row sees the
    // key tiles (and the products) of the 128-row form and attn_gqa_kernel.
    const bool wide = k.nsplit == 1 && plane_rows_wide(n, k.group, k.n_kv_heads);
    const int qt = (wide ? kPlaneRowsWide : kGqaRows) / k.group;
    dim3 grid((unsigned)((n + qt - 1) / qt), (unsigned)k.n_kv_heads, (unsigned)k.nsplit);
    if (grid.x > 0xffff || grid.y > 0xffff || k.n_heads > 0x7fff) return hipErrorInvalidValue;
    const int gxy = (int)(grid.x | grid.y << 16), gnh = k.group | k.n_heads << 16;
    if (wide)
        attn_planes_kernel<kPlaneWaves, kPlaneRowsWide><<<grid, 64 * kPlaneWaves, 0, s>>>(gxy, (int)n, gnh, k.q, k, pr);
    else
        attn_planes_kernel<kPlaneWaves, kGqaRows><<<grid, 64 * kPlaneWaves, 0, s>>>(gxy, (int)n, gnh, k.q, k, pr);
    e = hipGetLastError();
    if (e != hipSuccess || k.nsplit == 1) return e;
    return launch_attn_combine(s, k.out, k.part_acc, k.part_ml, n * (size_t)k.n_heads, k.nsplit, 128, k.out_hi,
                               k.out_lo);
}

}  // namespace th
