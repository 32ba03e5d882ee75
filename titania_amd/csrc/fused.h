// Fused forward-pass kernels and the device-resident state of the greedy decode loop.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "device_util.h"

namespace th {

// Arguments of the per-head q/k-norm + RoPE + KV append kernel. Caches are
// addressed as base + head * head_stride + position * pos_stride (elements).
struct QkvPostArgs {
    float *q;        // [n][n_heads][head_dim], normalized and rotated in place
    const float *k;  // [n][n_kv_heads][head_dim]
    const float *v;  // [n][n_kv_heads][head_dim]
    const uint16_t *q_norm, *k_norm;  // per-head gains, or null for none
    const float *rope;                // [max_len][head_dim/2][cos, sin]
    void *k_cache, *v_cache;
    long long head_stride, pos_stride;
    long long pos;
    const long long *pos_dev;  // position from device memory when not null
    int n, n_heads, n_kv_heads, head_dim;
    int kv_bf16;
    float eps;
    // When not null (f32 caches, head_dim 128): the prefill attention's bf16
    // planes of the new keys and values, written beside the caches: K hi / lo
    // [n_kv_heads][plane_len][128], V^T hi / lo [n_kv_heads][128][plane_len]
    // with each 32-key slice in the order of vt_column.
    uint16_t *kh, *kl, *vh, *vl;
    long long plane_len;
};

hipError_t launch_qk_norm_rope_append(hipStream_t s, const QkvPostArgs &a);

// The column of key k (0..31) within a 32-key slice of a V^T plane: the
// slice's column 8 g + i holds key 4 g + i for i < 4 and 16 + 4 g + i - 4
// otherwise (g < 4), the order in which the prefill attention's P^T operand
// meets the keys.
__host__ __device__ __forceinline__ int vt_column(int k) { return 8 * ((k & 15) >> 2) + ((k >> 4) << 2) + (k & 3); }

// State of the on-device greedy loop, in device memory so that one captured
// decode step can replay at every position.
constexpr int kStepMaxStops = 8;  // stop tokens a decode call may end at

struct StepState {
    long long pos;         // position of the token to feed next
    long long step;        // tokens fed so far in this decode call
    uint32_t token;        // token to feed next
    uint32_t epoch;        // decode steps ever advanced on this state (tags exchange words)
    uint32_t *tokens_out;  // picks, indexed by step
    float *logits_out;     // logits after each fed token, or null
    int n_stop;            // entries of stop[] in use
    int stopped;           // index in tokens_out of the stop token picked, plus one (0: none yet)
    uint32_t stop[kStepMaxStops];
};

// The embedding row the pick writes for the next step (model/cpu.rs:38-47),
// when `table` is not null: out[0..dim) = bf16 -> f32 of table[token].
struct PickEmbed {
    const uint16_t *table = nullptr;
    size_t dim = 0;
    float *out = nullptr;
};

// Records the step's pick and returns the token the next step feeds. With
// `advance` (a token has been fed) the position, step and epoch move on
// first; then st->token and st->tokens_out[st->step]. A pick in stop[] is
// recorded after the others but not fed (model/chat.rs:149-153): the position
// stays on the last fed token, which later steps of the call feed again at
// that position, rewriting the same cache row and logits, and their picks are
// dropped. The epoch advances with every step all the same, so that the
// exchange words of each step carry a tag of their own.
__device__ __forceinline__ uint32_t step_record(StepState *st, int advance, uint32_t tok) {
    if (advance) st->epoch += 1;
    if (st->stopped) return st->token;
    bool stop = false;
    for (int i = 0; i < st->n_stop; ++i) stop = stop || tok == st->stop[i];
    if (stop) {
        const long long at = st->step + (advance ? 1 : 0);
        if (st->tokens_out) st->tokens_out[at] = tok;
        st->stopped = (int)at + 1;
        return st->token;
    }
    if (advance) {
        st->pos += 1;
        st->step += 1;
    }
    st->token = tok;
    if (st->tokens_out) st->tokens_out[st->step] = tok;
    return tok;
}

// step_record from a copy of the state read ahead (`loc`, loaded before the
// caller's own loads, so that its round trip overlaps theirs instead of
// following its pick), writing back only the fields that change; the same
// updates as step_record when nothing else writes the state meanwhile.
__device__ __forceinline__ uint32_t step_record_from(StepState *st, const StepState &loc, int advance, uint32_t tok) {
    if (advance) st->epoch = loc.epoch + 1;
    if (loc.stopped) return loc.token;
    bool stop = false;
#pragma unroll
    for (int i = 0; i < kStepMaxStops; ++i) stop = stop || (i < loc.n_stop && tok == loc.stop[i]);
    const long long step = loc.step + (advance ? 1 : 0);
    if (stop) {
        if (loc.tokens_out) loc.tokens_out[step] = tok;
        st->stopped = (int)step + 1;
        return loc.token;
    }
    if (advance) {
        st->pos = loc.pos + 1;
        st->step = step;
    }
    st->token = tok;
    if (loc.tokens_out) loc.tokens_out[step] = tok;
    return tok;
}

// emb.out = the embedding row of `tok` (model/cpu.rs:38-47), by the block.
__device__ __forceinline__ void write_embedding(const PickEmbed &emb, uint32_t tok) {
    const uint4 *row = reinterpret_cast<const uint4 *>(emb.table + (size_t)tok * emb.dim);
    for (size_t c = threadIdx.x; c < emb.dim / 8; c += blockDim.x) {
        float f[8];
        unpack8(row[c], f);
        float4 *o = reinterpret_cast<float4 *>(emb.out + c * 8);
        o[0] = make_float4(f[0], f[1], f[2], f[3]);
        o[1] = make_float4(f[4], f[5], f[6], f[7]);
    }
}

// argmax of the logits -> st->token and st->tokens_out[st->step]; with
// `advance`, pos and step move on first.
hipError_t launch_pick(hipStream_t s, const float *logits, size_t vocab, uint64_t *partials, StepState *st,
                       int advance, const PickEmbed &emb = PickEmbed());
// The pick from per-block (key, inverted index) maxima already reduced by a kernel.
hipError_t launch_pick_partials(hipStream_t s, const uint64_t *partials, size_t m, StepState *st, int advance,
                                const PickEmbed &emb = PickEmbed());
hipError_t launch_keep_logits(hipStream_t s, const float *logits, size_t vocab, const StepState *st);

__device__ __forceinline__ void store_kv(float *p, float v) { *p = v; }
__device__ __forceinline__ void store_kv(uint16_t *p, float v) { *p = f32_to_bf16(v); }

// The q/k post-processing of one (token, head) row of head_dim <= 512 by a
// wave: lane i holds the RoPE pairs (i + 64 k, i + 64 k + head_dim/2) in
// av[k], bv[k] (zero past head_dim/2). RMSNorm of the row with `gain` (if not
// null; model/cpu.rs:85-94) and the rotation by the table row `ang`
// (model/cpu.rs:96-111), in registers. The post kernel and the q/k/v GEMM's
// epilogue share it, so both paths round alike.
__device__ __forceinline__ void norm_rope_pairs(float av[4], float bv[4], int lane, int hd, const uint16_t *gain,
                                                float eps, const float *ang) {
    const int half = hd / 2;
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) ss += av[k] * av[k] + bv[k] * bv[k];
    if (gain) {
        ss = wave_sum(ss);
        const float scale = 1.0f / sqrtf(ss / (float)hd + eps);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = lane + 64 * k;
            if (i < half) {
                av[k] = av[k] * (scale * bf16_to_f32(gain[i]));
                bv[k] = bv[k] * (scale * bf16_to_f32(gain[i + half]));
            }
        }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int i = lane + 64 * k;
        if (i < half) {
            const float c = ang[2 * i], sn = ang[2 * i + 1];
            const float x0 = av[k] * c - bv[k] * sn;
            const float x1 = bv[k] * c + av[k] * sn;
            av[k] = x0;
            bv[k] = x1;
        }
    }
}

}  // namespace th
