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

// Where kStore writes row r.
__device__ __forceinline__ float *store_at(const GemvArgs &a, int r) {
    if (!a.outs[0]) return a.out + r;
    if (r < a.rows.count[0]) return a.outs[0] + r;
    r -= a.rows.count[0];
    if (r < a.rows.count[1]) return a.outs[1] + r;
    return a.outs[2] + (r - a.rows.count[1]);
}

// One block: RPW rows per wave, CPL 16-byte chunks per lane per row.
template <int RPW, int CPL, Prologue PRO, Epilogue EPI>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvArgs a) {
    static_assert(EPI != kSiluPairs || RPW % 2 == 0, "a wave holds whole (gate, up) pairs");
    extern __shared__ float xs[];
    __shared__ float red[kWaves];
    __shared__ uint64_t red64[kWaves];
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    constexpr int RPB = RPW * kWaves;
    const int r0 = blockIdx.x * RPB + wave * RPW;
    // For paired rows (gate j, up j), a wave takes j and j + half.
    const int half = a.n_rows / 2;
    uint4 w[RPW][CPL];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        int row;
        if (EPI == kSiluPairs) row = (r & 1) ? (r0 + r - 1) / 2 + half : (r0 + r) / 2;
        else row = r0 + r;
        const bool valid = EPI == kSiluPairs ? (r0 + r - (r & 1)) / 2 < half : row < a.n_rows;
        const uint4 *p = row_at(a.rows, valid ? row : 0, a.cols);
#pragma unroll
        for (int c = 0; c < CPL; ++c) w[r][c] = ld_nt_row(p, c * 64 + lane);
    }
    build_input<PRO == kNormSum, (CPL * 128 + kThreads - 1) / kThreads>(xs, a.a, a.b, a.cols, a.gain, a.eps, a.x_out,
                                                                        red);
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
                if (lane == r && r0 + r < a.n_rows) *store_at(a, r0 + r) = res[r];
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
            if (r0 + r < a.n_rows) {
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

template <int RPW, int CPL, Prologue PRO, Epilogue EPI>
hipError_t gemv_launch(hipStream_t s, const GemvArgs &a) {
    constexpr int RPB = RPW * kWaves;
    dim3 grid((unsigned)((a.n_rows + RPB - 1) / RPB));
    gemv_kernel<RPW, CPL, PRO, EPI><<<grid, kThreads, a.cols * sizeof(float), s>>>(a);
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
        return gemv_launch<(RPW > 1 && EPI != kSiluPairs ? 1 : RPW), 19, PRO, EPI>(s, a);
    default: return hipErrorInvalidValue;
    }
}

// ---- attention for one token: q/k RMSNorm + RoPE + KV append + split attention ----

constexpr int kStageRows = 64;  // cached positions staged in LDS per pass

__device__ __forceinline__ void dma16(const void *src, void *wave_base) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)wave_base, 16, 0, 0);
}

__device__ __forceinline__ float lds_at(const float *row, int d) { return row[d]; }
__device__ __forceinline__ float lds_at(const uint16_t *row, int d) { return bf16_to_f32(row[d]); }

// Attention of one (KV head g, split of the positions 0..pos) by one block:
// the group's q heads and the new k are RMSNorm'd and rotated in LDS, the split
// holding pos appends k and v to the caches, and cached K/V rows are staged
// into LDS 64 positions at a time (all loads of a pass in flight together) for
// scores, online softmax and the weighted sum of values.
//
// The raw q/k/v come from a.qkv, or (WORDS) from (value | epoch << 32) words
// that other blocks of the same launch are writing: then the block first
// stages the cached rows (they do not depend on the q/k/v), then polls until
// every word it needs carries `epoch` (bounded: about 2 s, then *err counts
// the failure and the block goes on with what it has).
template <int HD, int G, typename KV, bool WORDS, int ROWS>
__device__ __forceinline__ void attend(const StepAttnArgs &a, int g, int split, const unsigned long long *words,
                                       unsigned epoch, unsigned *err) {
    constexpr int LPK = HD / 8, KPW = 64 / LPK, KPB = kWaves * KPW, NP = kThreads / HD;
    static_assert(LPK == 16, "one key per 16-lane row");
    constexpr int ROW16 = HD * (int)sizeof(KV) / 16;  // 16-byte chunks per cached row
    __shared__ float hq[G * HD], hk[HD], hv[HD];
    __shared__ float scores[G][ROWS];
    __shared__ float st_m[G], st_l[G], st_a[G];
    __shared__ float red[G][kThreads];
    __shared__ uint4 kst[ROWS * ROW16], vst[ROWS * ROW16];
    static_assert(HD == 128, "one rotation pair per lane");
    constexpr int HALF = HD / 2, HPW = (G + 1 + kWaves - 1) / kWaves;  // heads (q..., k) per wave
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, sub = lane % LPK;
    const int qd = a.n_heads * HD, kvd = a.n_kv_heads * HD;
    const KV *kc = reinterpret_cast<const KV *>(a.k_cache) + (size_t)g * a.head_stride;
    const KV *vc = reinterpret_cast<const KV *>(a.v_cache) + (size_t)g * a.head_stride;
    auto stage = [&](long long c0, int rows) {
        const int chunks = rows * ROW16;
        const uint4 *ks = reinterpret_cast<const uint4 *>(kc + c0 * HD);
        const uint4 *vs = reinterpret_cast<const uint4 *>(vc + c0 * HD);
        for (int base = wave * 64; base < chunks; base += kThreads)
            if (base + lane < chunks) {
                dma16(ks + base + lane, kst + base);
                dma16(vs + base + lane, vst + base);
            }
    };
    // The raw q heads and k of this wave (lane holds the pair (lane, lane +
    // HD/2)), their RMSNorm gains and this thread's element of v; from a.qkv
    // they are requested first, with everything else that does not depend on
    // the position.
    float av[HPW], bv[HPW], ga[HPW], gb[HPW];
    float vnew = 0.f;
#pragma unroll
    for (int hh = 0; hh < HPW; ++hh) {
        const int h = wave + hh * kWaves;
        av[hh] = bv[hh] = 0.f;
        ga[hh] = gb[hh] = 1.f;
        if (h <= G) {
            const uint16_t *gain = h < G ? a.q_norm : a.k_norm;
            if (gain) {
                ga[hh] = bf16_to_f32(gain[lane]);
                gb[hh] = bf16_to_f32(gain[lane + HALF]);
            }
            if (!WORDS) {
                const float *x = h < G ? a.qkv + (size_t)(g * G + h) * HD : a.qkv + qd + (size_t)g * HD;
                av[hh] = x[lane];
                bv[hh] = x[lane + HALF];
            }
        }
    }
    if (!WORDS && tid < HD) vnew = a.qkv[qd + kvd + (size_t)g * HD + tid];
    const long long pos = *a.pos;
    const long long len = pos + 1;
    const long long chunk = ((len + a.nsplit - 1) / a.nsplit + 15) / 16 * 16;
    const long long s0 = (long long)split * chunk;
    const long long s1 = s0 + chunk < len ? s0 + chunk : len;
    auto cached_in = [&](long long c0, int cnt) -> int {
        const long long nc = pos - c0;
        return nc <= 0 ? 0 : (nc < cnt ? (int)nc : cnt);
    };
    // Then, once pos is known, the rotation of this position and the first
    // pass's cached rows: one more memory round trip.
    const float2 cs = reinterpret_cast<const float2 *>(a.rope + pos * HD)[lane];
    {
        const int cnt0 = (int)(s1 - s0 < ROWS ? s1 - s0 : ROWS);
        if (s0 < s1) stage(s0, cached_in(s0, cnt0));
    }
    if (WORDS) {
        for (int it = 0;; ++it) {
            int ok = 1;
            unsigned long long wa[HPW], wb[HPW], wv = 0;
#pragma unroll
            for (int hh = 0; hh < HPW; ++hh) {
                const int h = wave + hh * kWaves;
                if (h <= G) {
                    const unsigned long long *x = h < G ? words + (size_t)(g * G + h) * HD : words + qd + (size_t)g * HD;
                    wa[hh] = __hip_atomic_load(x + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    wb[hh] = __hip_atomic_load(x + lane + HALF, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            if (tid < HD)
                wv = __hip_atomic_load(words + qd + kvd + (size_t)g * HD + tid, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int hh = 0; hh < HPW; ++hh) {
                const int h = wave + hh * kWaves;
                if (h <= G) {
                    ok &= (unsigned)(wa[hh] >> 32) == epoch && (unsigned)(wb[hh] >> 32) == epoch;
                    av[hh] = __uint_as_float((unsigned)wa[hh]);
                    bv[hh] = __uint_as_float((unsigned)wb[hh]);
                }
            }
            if (tid < HD) {
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
    // RMSNorm (model.rs:111-116) + RoPE (model.rs:117-118) per head, in registers.
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
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    float qf[G][8];
#pragma unroll
    for (int gg = 0; gg < G; ++gg)
#pragma unroll
        for (int i = 0; i < 8; ++i) qf[gg][i] = hq[gg * HD + sub * 8 + i];
    const float scale = 1.0f / sqrtf((float)HD);
    const int d = tid % HD, pt = tid / HD;
    const KV *ks_l = reinterpret_cast<const KV *>(kst), *vs_l = reinterpret_cast<const KV *>(vst);
    float acc[G];
#pragma unroll
    for (int gg = 0; gg < G; ++gg) acc[gg] = 0.f;
    for (long long c0 = s0; c0 < s1; c0 += ROWS) {
        const int cnt = (int)(s1 - c0 < ROWS ? s1 - c0 : ROWS);
        const int ncache = cached_in(c0, cnt);
        if (c0 != s0) {
            stage(c0, ncache);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        }
        for (int j0 = 0; j0 < cnt; j0 += KPB) {
            const int j = j0 + wave * KPW + lane / LPK;
            float kf[8];
            if (j < ncache) {
                lds_row8(ks_l + j * HD, sub, kf);
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) kf[i] = j < cnt ? hk[sub * 8 + i] : 0.f;
            }
#pragma unroll
            for (int gg = 0; gg < G; ++gg) {
                float sc = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) sc = fmaf(qf[gg][i], kf[i], sc);
                sc = row_sum_dpp(sc);
                if (j < cnt && sub == 0) scores[gg][j] = scale * sc;
            }
        }
        __syncthreads();
        for (int gg = wave; gg < G; gg += kWaves) {
            float m = -INFINITY;
            for (int j = lane; j < cnt; j += 64) m = fmaxf(m, scores[gg][j]);
            m = wave_max_dpp(m);
            const float m_old = st_m[gg], m_new = fmaxf(m_old, m);
            float l = 0.f;
            for (int j = lane; j < cnt; j += 64) {
                const float e = expf(scores[gg][j] - m_new);
                scores[gg][j] = e;
                l += e;
            }
            l = wave_sum_dpp(l);
            if (lane == 0) {
                const float al = expf(m_old - m_new);
                st_a[gg] = al;
                st_l[gg] = st_l[gg] * al + l;
                st_m[gg] = m_new;
            }
        }
        __syncthreads();
#pragma unroll
        for (int gg = 0; gg < G; ++gg) acc[gg] *= st_a[gg];
        for (int j = pt; j < cnt; j += NP) {
            const float v = j < ncache ? lds_at(vs_l + j * HD, d) : hv[d];
#pragma unroll
            for (int gg = 0; gg < G; ++gg) acc[gg] = fmaf(scores[gg][j], v, acc[gg]);
        }
        __syncthreads();  // the stage and scores are rewritten by the next pass
    }
    // The split holding pos appends the new key and value (model.rs:119-120);
    // no block of this launch reads that position from the caches.
    if (pos >= s0 && pos < s1 && tid < HD) {
        KV *kw = reinterpret_cast<KV *>(a.k_cache) + (size_t)g * a.head_stride + pos * HD;
        KV *vw = reinterpret_cast<KV *>(a.v_cache) + (size_t)g * a.head_stride + pos * HD;
        store_kv(kw + tid, hk[tid]);
        store_kv(vw + tid, hv[tid]);
    }
#pragma unroll
    for (int gg = 0; gg < G; ++gg) red[gg][tid] = acc[gg];
    __syncthreads();
    if (pt != 0) return;
    for (int gg = 0; gg < G; ++gg) {
        float sm = red[gg][d];
        for (int q = 1; q < NP; ++q) sm += red[gg][q * HD + d];
        const long long h = (long long)g * G + gg;
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

template <int HD, int G, typename KV>
__global__ __launch_bounds__(kThreads) void step_attention_kernel(StepAttnArgs a) {
    attend<HD, G, KV, false, kStageRows>(a, blockIdx.x / a.nsplit, blockIdx.x % a.nsplit, nullptr, 0, nullptr);
}

// The q/k/v rows of launch_step_qkv (kQkvRowsPerWave per wave) published as
// epoch words by the first blocks, and after them one block per q head and
// chunk of the cache that attends from those words. Blocks start in index order and the GEMV blocks never wait, so
// the attention blocks' polls always end.
// Rows a wave of the q/k/v GEMV blocks in qkv_attn_kernel (Qwen3-0.6B step:
// 0.6114 ms with 2, 0.6094 with 4, 0.645 with 1; with the branch-free P.V
// loop, 0.5990 with 4 and 0.5975 with 5; with non-temporal weight loads,
// 0.5673 / 0.5651 / 0.5640 / 0.5693 ms with 2 / 3 / 4 / 5).
constexpr int kQkvRowsPerWave = 4;

template <int CPL, int G, typename KV>
__global__ __launch_bounds__(kThreads) void qkv_attn_kernel(StepQkvAttnArgs q, GemvArgs a) {
    constexpr int RPW = kQkvRowsPerWave, RPB = RPW * kWaves;
    const int ngemv = (a.n_rows + RPB - 1) / RPB;
    const unsigned epoch = q.st->epoch * 64u + (unsigned)q.layer + 1u;
    if ((int)blockIdx.x >= ngemv) {
        // `chunks` blocks per q head, one per pass of cached rows: the heads
        // of a KV group attend in parallel (each reads the group's rows), the
        // group's first head appends; each head's first chunk merges.
        const int b = blockIdx.x - ngemv, h = b / q.chunks, c = b % q.chunks, g = h / G;
        unsigned long long *xw = q.words + q.qkv.q_rows + 2 * q.qkv.kv_rows;
        attend_wave4<KV>(q.at, g, h, h % G == 0, c, q.words, epoch, q.err, xw, q.chunks);
        return;
    }
    extern __shared__ float xs[];
    __shared__ float red[kWaves];
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int r0 = blockIdx.x * RPB + wave * RPW;
    uint4 w[RPW][CPL];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const uint4 *p = row_at(a.rows, r0 + r < a.n_rows ? r0 + r : 0, a.cols);
#pragma unroll
        for (int c = 0; c < CPL; ++c) w[r][c] = ld_nt_row(p, c * 64 + lane);
    }
    build_input<true, (CPL * 128 + kThreads - 1) / kThreads>(xs, a.a, a.b, a.cols, a.gain, a.eps, a.x_out, red);
    float res[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) acc = dot8(xs, w[r][c], c * 64 + lane, acc);
        res[r] = wave_sum_dpp(acc);
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r)
        if (lane == r && r0 + r < a.n_rows)
            __hip_atomic_store(q.words + r0 + r, ((unsigned long long)epoch << 32) | __float_as_uint(res[r]),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int CPL, int G>
hipError_t qkv_attn_launch(hipStream_t s, const StepQkvAttnArgs &q, const GemvArgs &a) {
    constexpr int RPB = kQkvRowsPerWave * kWaves;
    dim3 grid((unsigned)((a.n_rows + RPB - 1) / RPB + q.at.n_heads * q.chunks));
    const size_t lds = (size_t)a.cols * sizeof(float);
    if (q.at.kv_bf16)
        qkv_attn_kernel<CPL, G, uint16_t><<<grid, kThreads, lds, s>>>(q, a);
    else
        qkv_attn_kernel<CPL, G, float><<<grid, kThreads, lds, s>>>(q, a);
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

// One block per (KV head, split of `chunk` positions), cached rows in
// registers; at most 168 VGPRs, so that three blocks fit on a CU.
template <int G, typename KV>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3)))
void step_attention_regs_kernel(StepAttnArgs a, long long chunk) {
    const int g = blockIdx.x / a.nsplit;
    attend_regs<G, KV, false>(a, g, g * G, true, blockIdx.x % a.nsplit, chunk, nullptr, 0, nullptr);
}

template <int G>
hipError_t attn_regs_launch(hipStream_t s, const StepAttnArgs &a) {
    const long long max_len = a.head_stride / 128;
    const int rows = a.kv_bf16 ? KvRegs<uint16_t>::kRows : KvRegs<float>::kRows;
    long long chunk = (max_len + a.nsplit - 1) / a.nsplit;
    chunk = (chunk + rows - 1) / rows * rows;
    dim3 grid((unsigned)(a.n_kv_heads * a.nsplit));
    if (a.kv_bf16)
        step_attention_regs_kernel<G, uint16_t><<<grid, kThreads, 0, s>>>(a, chunk);
    else
        step_attention_regs_kernel<G, float><<<grid, kThreads, 0, s>>>(a, chunk);
    return hipGetLastError();
}

template <int HD, int G>
hipError_t attn_launch(hipStream_t s, const StepAttnArgs &a) {
    dim3 grid((unsigned)(a.n_kv_heads * a.nsplit));
    if (a.kv_bf16)
        step_attention_kernel<HD, G, uint16_t><<<grid, kThreads, 0, s>>>(a);
    else
        step_attention_kernel<HD, G, float><<<grid, kThreads, 0, s>>>(a);
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
    return gemv_dispatch<2, kNormSum, kStore>(s, a);
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

size_t step_qkv_attn_words(int q_rows, int kv_rows, int n_heads, int chunks) {
    return (size_t)q_rows + 2 * (size_t)kv_rows + (size_t)n_heads * chunks * (128 + 2);
}

hipError_t launch_step_qkv_attn(hipStream_t s, const StepQkvAttnArgs &q) {
    const StepQkvArgs &k = q.qkv;
    const long long max_len = q.at.head_stride / 128;
    if (!step_qkv_attn_supported(k.hidden, q.at.n_heads, q.at.n_kv_heads) || q.at.nsplit != 1 || q.chunks < 1 ||
        q.chunks != step_qkv_attn_chunks((size_t)max_len, q.at.kv_bf16, q.at.n_heads))
        return hipErrorInvalidValue;
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
    switch (k.hidden / 512) {
    case 1: return qkv_attn_g<1>(s, q, a);
    case 2: return qkv_attn_g<2>(s, q, a);
    case 5: return qkv_attn_g<5>(s, q, a);
    default: return hipErrorInvalidValue;
    }
}

int step_attention_splits(size_t max_len, int kv_bf16) {
    if (max_len <= 512) return 1;
    const size_t rows = kv_bf16 ? KvRegs<uint16_t>::kRows : KvRegs<float>::kRows;
    return (int)std::min<size_t>((max_len + rows - 1) / rows, 256);
}

hipError_t launch_step_attention(hipStream_t s, const StepAttnArgs &a) {
    switch (a.n_heads / a.n_kv_heads) {
    case 1: return attn_launch<128, 1>(s, a);
    case 2: return attn_regs_launch<2>(s, a);
    case 4: return attn_regs_launch<4>(s, a);
    case 8: return attn_launch<128, 8>(s, a);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace th
