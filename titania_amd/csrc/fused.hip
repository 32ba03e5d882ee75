// Fused kernels of the forward pass: per-head q/k RMSNorm + RoPE + KV-cache
// append in one launch, and the greedy-decode bookkeeping that keeps the token
// loop on the device.
#include "common.h"
#include "device_util.h"
#include "fused.h"

namespace th {

// One wave per (token, head) over the n_heads query heads followed by the
// n_kv_heads key heads. Each lane holds RoPE pairs (i, i + head_dim/2), so the
// head's RMSNorm (model/cpu.rs:85-94, rows of head_dim) and its rotation
// (model/cpu.rs:96-111) happen in registers. Query heads are written back in
// place; key heads, and the value heads beside them, go to the caches at
// position pos + t (model/model.rs:111-120).
template <typename KV>
__global__ __launch_bounds__(256) void qk_norm_rope_append_kernel(QkvPostArgs a) {
    const int lane = threadIdx.x & 63;
    const long long item = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int heads = a.n_heads + a.n_kv_heads;
    if (item >= (long long)a.n * heads) return;
    const long long t = item / heads;
    const int h = (int)(item % heads);
    const long long pos = (a.pos_dev ? *a.pos_dev : a.pos) + t;
    const int hd = a.head_dim, half = hd / 2;
    const bool is_q = h < a.n_heads;
    const float *src = is_q ? a.q + (t * a.n_heads + h) * hd : a.k + (t * a.n_kv_heads + (h - a.n_heads)) * hd;
    const uint16_t *gain = is_q ? a.q_norm : a.k_norm;

    // Pairs i = lane, lane + 64, ... (at most 4 per lane: head_dim <= 512).
    float av[4], bv[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        int i = lane + 64 * k;
        av[k] = i < half ? src[i] : 0.f;
        bv[k] = i < half ? src[i + half] : 0.f;
    }
    norm_rope_pairs(av, bv, lane, hd, gain, a.eps, a.rope + pos * hd);
    if (is_q) {
        float *dst = a.q + (t * a.n_heads + h) * hd;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            int i = lane + 64 * k;
            if (i < half) {
                dst[i] = av[k];
                dst[i + half] = bv[k];
            }
        }
        return;
    }
    const int g = h - a.n_heads;
    KV *kc = reinterpret_cast<KV *>(a.k_cache) + (long long)g * a.head_stride + pos * a.pos_stride;
    KV *vc = reinterpret_cast<KV *>(a.v_cache) + (long long)g * a.head_stride + pos * a.pos_stride;
    const float *vsrc = a.v + (t * a.n_kv_heads + g) * hd;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        int i = lane + 64 * k;
        if (i < half) {
            store_kv(kc + i, av[k]);
            store_kv(kc + i + half, bv[k]);
            store_kv(vc + i, vsrc[i]);
            store_kv(vc + i + half, vsrc[i + half]);
        }
    }
}

hipError_t launch_qk_norm_rope_append(hipStream_t s, const QkvPostArgs &a) {
    if (a.n == 0) return hipSuccess;
    long long items = (long long)a.n * (a.n_heads + a.n_kv_heads);
    dim3 grid((unsigned)((items + 3) / 4));
    if (a.kv_bf16)
        qk_norm_rope_append_kernel<uint16_t><<<grid, 256, 0, s>>>(a);
    else
        qk_norm_rope_append_kernel<float><<<grid, 256, 0, s>>>(a);
    return hipGetLastError();
}

// Greedy pick of the decode loop: reduces the argmax partials, records the
// token as the step's pick and as the next token to feed, and advances the
// position when `advance` is set (after a token has been fed).
__global__ __launch_bounds__(1024) void pick_kernel(const uint64_t *__restrict__ partials, size_t m, StepState *st,
                                                   int advance, PickEmbed emb) {
    __shared__ uint64_t red[16];
    __shared__ uint32_t picked;
    // The state, read before the partials (its wait then ends with theirs).
    StepState loc{};
    if (threadIdx.x == 0) loc = *st;
    uint64_t best = 0;
    // Sixteen loads in flight per thread per round: the 9496 partials of a
    // 151936-entry vocabulary in one round trip (with eight a round, two
    // dependent ones).
    for (size_t i0 = threadIdx.x; i0 < m; i0 += 16 * 1024) {
        uint64_t v[16];
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] = i0 + k * 1024 < m ? partials[i0 + k * 1024] : 0;
#pragma unroll
        for (int k = 0; k < 16; ++k) best = max_u64(best, v[k]);
    }
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = 0;
        for (int w = 0; w < 16; ++w) b = max_u64(b, red[w]);
        picked = step_record_from(st, loc, advance, argmax_index(b));
    }
    if (!emb.table) return;
    __syncthreads();
    write_embedding(emb, picked);
}

// Copies the logits into row `step` of the caller's logits array (the logits
// after the token fed at this step), when the caller asked for them.
__global__ void keep_logits_kernel(const float *__restrict__ logits, size_t vocab, const StepState *st) {
    if (!st->logits_out) return;
    float *dst = st->logits_out + (size_t)st->step * vocab;
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < vocab; i += stride) dst[i] = logits[i];
}

hipError_t launch_pick(hipStream_t s, const float *logits, size_t vocab, uint64_t *partials, StepState *st,
                       int advance, const PickEmbed &emb) {
    if (emb.table && emb.dim % 8) return hipErrorInvalidValue;
    size_t m = argmax_partials(vocab);
    hipError_t e = launch_argmax_partials(s, logits, vocab, partials);
    if (e != hipSuccess) return e;
    pick_kernel<<<1, 1024, 0, s>>>(partials, m, st, advance, emb);
    return hipGetLastError();
}

hipError_t launch_pick_partials(hipStream_t s, const uint64_t *partials, size_t m, StepState *st, int advance,
                                const PickEmbed &emb) {
    if (emb.table && emb.dim % 8) return hipErrorInvalidValue;
    pick_kernel<<<1, 1024, 0, s>>>(partials, m, st, advance, emb);
    return hipGetLastError();
}

hipError_t launch_keep_logits(hipStream_t s, const float *logits, size_t vocab, const StepState *st) {
    keep_logits_kernel<<<64, 256, 0, s>>>(logits, vocab, st);
    return hipGetLastError();
}

}  // namespace th
