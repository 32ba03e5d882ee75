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
constexpr size_t kAttnTileMin = 8; // tokens from which a launch uses the query-tiled kernel
constexpr size_t kMKTiles = 32;    // positions per key tile of that kernel

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

// Merges the splits of one (token, head): rescales each split's sum and
// accumulator by exp(m_split - m_max); empty splits (m = -inf) add nothing.
// Every split's statistics and accumulator rows are read in parallel (threads
// over splits, then over (dimension, group of splits)), not one after another.
constexpr int kCombineThreads = 256, kMaxSplits = 256;

__global__ __launch_bounds__(kCombineThreads) void attn_combine_kernel(float *__restrict__ out,
                                                                      const float *__restrict__ part_acc,
                                                                      const float *__restrict__ part_ml, int nsplit,
                                                                      int hd, uint16_t *__restrict__ hi,
                                                                      uint16_t *__restrict__ lo) {
    __shared__ float w[kMaxSplits];
    __shared__ float red[kCombineThreads / 64];
    __shared__ float acc_red[kCombineThreads];
    const long long th = blockIdx.x;  // token * n_heads + head
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *ml = part_ml + th * nsplit * 2;
    float m = -INFINITY;
    for (int s = tid; s < nsplit; s += kCombineThreads) m = fmaxf(m, ml[2 * s]);
    m = wave_max_dpp(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float l = 0.f;
    for (int s = tid; s < nsplit; s += kCombineThreads) {
        const float ms = ml[2 * s];
        const float ws = ms != -INFINITY ? expf(ms - m) : 0.f;
        w[s] = ws;
        l += ml[2 * s + 1] * ws;
    }
    l = wave_sum_dpp(l);
    if (lane == 0) red[wave] = l;
    __syncthreads();
    l = ((red[0] + red[1]) + red[2]) + red[3];
    // groups of splits per dimension: thread t takes dimension t % hd of the
    // splits s = t / hd, + groups, ...
    const int groups = hd < kCombineThreads ? kCombineThreads / hd : 1;
    for (int d0 = 0; d0 < hd; d0 += kCombineThreads) {
        const int d = d0 + tid % hd, grp = tid / hd;
        float acc = 0.f;
        if (d < hd && grp < groups) {
            const float *pa = part_acc + th * nsplit * hd + d;
#pragma unroll 8
            for (int s = grp; s < nsplit; s += groups) acc += pa[(size_t)s * hd] * w[s];
        }
        acc_red[tid] = acc;
        __syncthreads();
        if (grp == 0 && d < hd) {
            float sum = 0.f;
            for (int gi = 0; gi < groups; ++gi) sum += acc_red[gi * hd + tid % hd];
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
    float ms = -INFINITY, ls = 0.f;
    if (lane < nsplit) {
        const float2 v = reinterpret_cast<const float2 *>(part_ml + th * nsplit * 2)[lane];
        ms = v.x;
        ls = v.y;
    }
    const float m = wave_max_dpp(ms);
    const float ws = ms != -INFINITY ? expf(ms - m) : 0.f;
    const float l = wave_sum_dpp(ls * ws);
    const float *pa = part_acc + th * nsplit * HD + lane * D;
    float acc[D];
#pragma unroll
    for (int d = 0; d < D; ++d) acc[d] = 0.f;
#pragma unroll 4
    for (int sp = 0; sp < nsplit; ++sp) {
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

int attention_splits(size_t n, size_t n_kv_heads, size_t max_len, size_t head_dim) {
    // Several tokens on the matrix cores: split a query tile's keys so that
    // each split walks at least 4 key tiles, at most 8 splits.
    if (head_dim == 128 && n >= kAttnTileMin) {
        const size_t tiles = (max_len + kMKTiles - 1) / kMKTiles;
        return (int)std::min<size_t>(std::max<size_t>(tiles / 4, 1), 8);
    }
    // One split while a block's share is short; otherwise about two blocks per
    // CU, each split covering at least 64 positions.
    if (max_len <= 512) return 1;
    size_t blocks_per_split = n * n_kv_heads;
    size_t want = (512 + blocks_per_split - 1) / blocks_per_split;
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
    attn_combine_kernel<<<dim3((unsigned)heads), dim3(kCombineThreads), 0, s>>>(out, part_acc, part_ml, nsplit, hd,
                                                                                hi, lo);
    return hipGetLastError();
}

// Prefill (several tokens, head_dim 128): one block per (tile of QT
// consecutive tokens, query head). The block stages the tile's queries once and
// walks the KV head's positions in tiles of KT rows staged in LDS, so each key
// and value row is read once per query tile rather than once per token. Thread
// t scores key t % 32 against queries 4 (t / 32) .. +3, the 32 lanes of a
// half-wave that share those queries reduce the row statistics with shuffles
// (online softmax, the causal mask per query), and the same thread then
// accumulates dims 4 (t % 32) .. +3 of those queries' outputs. All arithmetic
// is f32.
constexpr int kQT = 32, kKT = 32;

__device__ __forceinline__ float4 load4(const float *p) { return *reinterpret_cast<const float4 *>(p); }
__device__ __forceinline__ float4 load4(const uint16_t *p) {
    const uint2 w = *reinterpret_cast<const uint2 *>(p);
    return make_float4(bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y));
}

template <typename KV>
__global__ __launch_bounds__(256) void attn_tile_kernel(AttnKernelArgs a, int n) {
    constexpr int HD = 128, QS = HD + 4;  // padded row stride of the Q and K tiles
    __shared__ float qs[kQT * QS];
    __shared__ float ks[kKT * QS];
    __shared__ float vs[kKT * HD];
    __shared__ float ps[kQT * kKT];
    const int tid = threadIdx.x;
    const int h = blockIdx.y, g = h / a.group;
    const int t0 = blockIdx.x * kQT;
    const int nq = n - t0 < kQT ? n - t0 : kQT;
    const long long pos = a.pos_dev ? *a.pos_dev : a.pos;
    for (int i = tid; i < kQT * HD / 4; i += 256) {
        const int row = i / (HD / 4), c4 = i % (HD / 4);
        const float4 v = row < nq ? load4(a.q + ((long long)(t0 + row) * a.n_heads + h) * HD + c4 * 4)
                                  : make_float4(0.f, 0.f, 0.f, 0.f);
        *reinterpret_cast<float4 *>(qs + row * QS + c4 * 4) = v;
    }
    const KV *kb = reinterpret_cast<const KV *>(a.k) + (long long)g * a.head_stride;
    const KV *vb = reinterpret_cast<const KV *>(a.v) + (long long)g * a.head_stride;
    const int j = tid & 31, qi0 = (tid >> 5) * 4, d0 = (tid & 31) * 4;
    float m[4], l[4], acc[4][4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        m[q] = -INFINITY;
        l[q] = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[q][e] = 0.f;
    }
    const long long last = pos + t0 + nq - 1;  // the last position a query of the tile attends
    // Key/value rows travel through registers one tile ahead: the loads of
    // tile c0 + KT are in flight while tile c0 is scored.
    constexpr int PER = kKT * HD / 4 / 256;  // float4 of K (and of V) per thread per tile
    float4 kr4[PER], vr4[PER];
    auto fetch = [&](long long c0) {
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int i = tid + u * 256, row = i / (HD / 4), c4 = i % (HD / 4);
            const long long p = c0 + row;
            kr4[u] = vr4[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (p <= last) {
                kr4[u] = load4(kb + p * a.pos_stride + c4 * 4);
                vr4[u] = load4(vb + p * a.pos_stride + c4 * 4);
            }
        }
    };
    fetch(0);
    for (long long c0 = 0; c0 <= last; c0 += kKT) {
        __syncthreads();  // the previous tile's rows are consumed (and the queries stored)
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int i = tid + u * 256, row = i / (HD / 4), c4 = i % (HD / 4);
            *reinterpret_cast<float4 *>(ks + row * QS + c4 * 4) = kr4[u];
            *reinterpret_cast<float4 *>(vs + row * HD + c4 * 4) = vr4[u];
        }
        __syncthreads();
        if (c0 + kKT <= last) fetch(c0 + kKT);
        float sc[4] = {0.f, 0.f, 0.f, 0.f};
        const float *kr = ks + j * QS;
#pragma unroll 8
        for (int c = 0; c < HD; c += 4) {
            const float4 kk = *reinterpret_cast<const float4 *>(kr + c);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 qv = *reinterpret_cast<const float4 *>(qs + (qi0 + q) * QS + c);
                sc[q] = fmaf(qv.x, kk.x, sc[q]);
                sc[q] = fmaf(qv.y, kk.y, sc[q]);
                sc[q] = fmaf(qv.z, kk.z, sc[q]);
                sc[q] = fmaf(qv.w, kk.w, sc[q]);
            }
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const long long qp = pos + t0 + qi0 + q;  // the query's position
            const bool valid = qi0 + q < nq && c0 + j <= qp;
            const float sv = valid ? a.scale * sc[q] : -INFINITY;
            float mx = sv;
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 32));
            const float mn = fmaxf(m[q], mx);
            const float pv = sv == -INFINITY ? 0.f : expf(sv - mn);
            float sum = pv;
#pragma unroll
            for (int o = 16; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 32);
            const float al = m[q] == -INFINITY ? 0.f : expf(m[q] - mn);
            l[q] = l[q] * al + sum;
            m[q] = mn;
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[q][e] *= al;
            ps[(qi0 + q) * kKT + j] = pv;
        }
        __syncthreads();
#pragma unroll 4
        for (int jj = 0; jj < kKT; ++jj) {
            const float4 v4 = *reinterpret_cast<const float4 *>(vs + jj * HD + d0);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float pj = ps[(qi0 + q) * kKT + jj];
                acc[q][0] = fmaf(pj, v4.x, acc[q][0]);
                acc[q][1] = fmaf(pj, v4.y, acc[q][1]);
                acc[q][2] = fmaf(pj, v4.z, acc[q][2]);
                acc[q][3] = fmaf(pj, v4.w, acc[q][3]);
            }
        }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
        if (qi0 + q < nq) {
            float4 o = make_float4(acc[q][0] / l[q], acc[q][1] / l[q], acc[q][2] / l[q], acc[q][3] / l[q]);
            *reinterpret_cast<float4 *>(a.out + ((long long)(t0 + qi0 + q) * a.n_heads + h) * HD + d0) = o;
        }
}

// Prefill on the matrix cores (head_dim 128): one block per (tile of 64
// consecutive tokens, query head), 16 tokens per wave. Key/value rows walk
// through LDS 32 positions at a time (loaded one tile ahead, as f32); each
// wave forms S = Q K^T for its 16 queries with v_mfma_f32_16x16x4f32 (f32
// products, f32 sums), applies the causal mask and the online softmax along
// its 16-lane rows, passes P through LDS into the A-operand layout and adds
// P V into 16 x 128 f32 accumulators. Layout of 16x16x4 (checked on the GPU):
// lane l holds A[l%16][l/16] and B[l/16][l%16], and D[4(l/16)+e][l%16].
constexpr int kMQT = 64, kMKT = (int)kMKTiles;
typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float row_max16(float v) {
    v = fmaxf(v, dpp_get<0xB1>(v, -INFINITY));
    v = fmaxf(v, dpp_get<0x4E>(v, -INFINITY));
    v = fmaxf(v, dpp_get<0x124>(v, -INFINITY));
    v = fmaxf(v, dpp_get<0x128>(v, -INFINITY));
    return v;
}

template <typename KV>
__global__ __launch_bounds__(256) void attn_mfma_kernel(AttnKernelArgs a, int n) {
    constexpr int HD = 128, KS = HD + 4, VS = HD + 16, PS = kMKT + 4;  // LDS row strides (floats)
    __shared__ float ks[kMKT * KS];
    __shared__ float vs[kMKT * VS];
    __shared__ float ps[4][16 * PS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int li = lane & 15, lk = lane >> 4;
    const int h = blockIdx.y, g = h / a.group;
    const int t0 = blockIdx.x * kMQT;
    const int nq = n - t0 < kMQT ? n - t0 : kMQT;
    const long long pos = a.pos_dev ? *a.pos_dev : a.pos;
    // Q in the A-operand layout: qa[k] = Q[query li of the wave][4k + lk].
    const int tq = t0 + wave * 16 + li;
    float qa[HD / 4];
    {
        const float *qp = a.q + ((long long)(tq < n ? tq : 0) * a.n_heads + h) * HD + lk;
#pragma unroll
        for (int k = 0; k < HD / 4; ++k) qa[k] = tq < n ? qp[4 * k] : 0.f;
    }
    const KV *kb = reinterpret_cast<const KV *>(a.k) + (long long)g * a.head_stride;
    const KV *vb = reinterpret_cast<const KV *>(a.v) + (long long)g * a.head_stride;
    const long long last = pos + t0 + nq - 1;                       // the block's last query position
    const long long wlast = pos + t0 + wave * 16 + 15;              // this wave's last query position
    // Key split z of a.nsplit: key tiles [kt0, kt1) of the block's range.
    const long long ntiles = last / kMKT + 1, z = blockIdx.z;
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
    constexpr int PER = kMKT * HD / 4 / 256;  // float4 of K (and of V) per thread per tile
    float4 kr4[PER], vr4[PER];
    auto fetch = [&](long long c0) {
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int i = tid + u * 256, row = i / (HD / 4), c4 = i % (HD / 4);
            const long long p = c0 + row;
            kr4[u] = vr4[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (p <= last) {
                kr4[u] = load4(kb + p * a.pos_stride + c4 * 4);
                vr4[u] = load4(vb + p * a.pos_stride + c4 * 4);
            }
        }
    };
    const long long cend = kt1 * kMKT;  // positions [kt0 kMKT, cend) of this split
    if (kt0 < kt1) fetch(kt0 * kMKT);
    for (long long c0 = kt0 * kMKT; c0 < cend; c0 += kMKT) {
        __syncthreads();  // the previous tile is consumed
#pragma unroll
        for (int u = 0; u < PER; ++u) {
            const int i = tid + u * 256, row = i / (HD / 4), c4 = i % (HD / 4);
            *reinterpret_cast<float4 *>(ks + row * KS + c4 * 4) = kr4[u];
            *reinterpret_cast<float4 *>(vs + row * VS + c4 * 4) = vr4[u];
        }
        __syncthreads();
        if (c0 + kMKT < cend) fetch(c0 + kMKT);
        if (c0 > wlast) continue;  // every query of this wave precedes the tile
        // S for keys c0 + [0, 16) and c0 + [16, 32).
        floatx4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < HD / 4; ++k) {
            const float b0 = ks[li * KS + 4 * k + lk], b1 = ks[(16 + li) * KS + 4 * k + lk];
            s0 = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[k], b0, s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[k], b1, s1, 0, 0, 0);
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
        // P back in the A-operand layout (same wave: LDS stays in order).
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        float pa[kMKT / 4];
#pragma unroll
        for (int kk = 0; kk < kMKT / 4; ++kk) pa[kk] = ps[wave][li * PS + 4 * kk + lk];
#pragma unroll
        for (int kk = 0; kk < kMKT / 4; ++kk)
#pragma unroll
            for (int d = 0; d < HD / 16; ++d)
                o[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[kk], vs[(4 * kk + lk) * VS + d * 16 + li], o[d], 0,
                                                            0, 0);
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
            // Unnormalised sum, max and denominator for launch_attn_combine
            // (a split with no key of this query leaves m = -inf).
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

template <int HD>
static hipError_t attn_launch(hipStream_t s, AttnKernelArgs k, size_t n) {
    dim3 grid((unsigned)(n * (size_t)k.n_kv_heads * (size_t)k.nsplit));
    if (k.kv_bf16)
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
        dim3 grid((unsigned)((n + kMQT - 1) / kMQT), (unsigned)k.n_heads, (unsigned)k.nsplit);
        if (k.kv_bf16)
            attn_mfma_kernel<uint16_t><<<grid, 256, 0, s>>>(k, (int)n);
        else
            attn_mfma_kernel<float><<<grid, 256, 0, s>>>(k, (int)n);
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

}  // namespace th
