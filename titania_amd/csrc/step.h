// Fused kernels of one greedy decode step (batch 1), for graph capture.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "device_util.h"
#include "fused.h"

namespace th {

// Whether the step kernels support this shape (head_dim 128, rows of whole
// 512-column spans).
bool step_supported(int hidden, int intermediate, int n_heads, int n_kv_heads, int head_dim);

struct StepQkvArgs {
    const uint16_t *wq, *wk, *wv;
    int q_rows, kv_rows, hidden;
    const float *x_prev, *y_prev;  // residual input: x_prev (+ y_prev)
    const uint16_t *gain;
    float eps;
    float *x_out;  // x_prev + y_prev
    float *qkv;    // [q rows][k rows][v rows]
};

// x_out = x_prev + y_prev; qkv = [Wq; Wk; Wv] . rmsnorm(x_out).
hipError_t launch_step_qkv(hipStream_t s, const StepQkvArgs &a);

// out = W . x for W [rows, cols].
hipError_t launch_step_gemv(hipStream_t s, const uint16_t *w, int rows, int cols, const float *x, float *out);

// Whether the step GEMVs take rows of `cols` columns (whole 512-column spans:
// 1-6, 8 or 19 of them).
bool step_gemv_supported(int cols);

// out[i] = w[i] . x for three matrices w[i] [rows[i], cols] in one launch.
hipError_t launch_step_gemv3(hipStream_t s, const uint16_t *const w[3], const int rows[3], int cols, const float *x,
                             float *const out[3]);

// h[j] = silu(gate_j . x) * (up_j . x) for j < inter (x already normalized).
hipError_t launch_step_silu(hipStream_t s, const uint16_t *gate, const uint16_t *up, int inter, int cols,
                            const float *x, float *h);

// x_out = x1 + o; h[j] = silu(gate_j . n) * (up_j . n) with n = rmsnorm(x_out).
hipError_t launch_step_gate_up(hipStream_t s, const uint16_t *gate, const uint16_t *up, int inter, int hidden,
                               const float *x1, const float *o, const uint16_t *gain, float eps, float *x_out,
                               float *h);

// logits = W . rmsnorm(x + y), and per-block argmax partials.
hipError_t launch_step_logits(hipStream_t s, const uint16_t *w, int vocab, int hidden, const float *x,
                              const float *y, const uint16_t *gain, float eps, float *logits, uint64_t *partials,
                              int *n_partials);
int step_logits_partials(int vocab);

struct StepAttnArgs {
    const float *qkv;  // raw q, k, v rows of the step (the q/k/v GEMV's output)
    const uint16_t *q_norm, *k_norm;  // or null
    const float *rope;                // [max_len][head_dim/2][cos, sin]
    void *k_cache, *v_cache;          // the layer's caches, [kv_head][max_len][head_dim]
    long long head_stride;            // max_len * head_dim
    const long long *pos;             // the step's position (device)
    int n_heads, n_kv_heads;
    int nsplit;
    int kv_bf16;
    float eps;
    float *out;       // [n_heads][head_dim] when nsplit == 1
    float *part_acc;  // [n_heads][nsplit][head_dim] otherwise
    float *part_ml;   // [n_heads][nsplit][2]
};

// Splits of the context launch_step_attention wants for caches of max_len
// positions, `group` q heads a KV head, on a GPU of num_cus compute units:
// one up to 512 positions, else as many as fill the chip's block slots in
// one round, in whole passes of its blocks (32 f32 / 64 bf16 positions), at
// most 256.
int step_attention_splits(size_t max_len, int kv_bf16, int group, int n_kv_heads, int num_cus);
// Block slots of the streaming attention's launches on a GPU of num_cus
// compute units (blocks a CU: the waves a SIMD it is built for).
int step_stream_slots(int group, int kv_bf16, int num_cus);
// Positions a split covers: max_len / nsplit rounded up to whole passes.
long long step_attention_chunk(size_t max_len, int kv_bf16, int nsplit);
hipError_t launch_step_attention(hipStream_t s, const StepAttnArgs &a);

// The q/k/v GEMV (as launch_step_qkv) and the attention in one launch: the
// GEMV blocks publish the rows as (value | epoch << 32) words, epoch =
// st->epoch * 64 + layer + 1; `chunks` extra blocks per q head, one per pass
// of cached rows, request their rows meanwhile, then attend from the words;
// the first chunk's block merges the others' partials (exchanged as words).
struct StepQkvAttnArgs {
    StepQkvArgs qkv;               // x_out as launch_step_qkv; qkv unused
    StepAttnArgs at;               // qkv and partials unused, nsplit 1
    // [q_rows + 2 kv_rows] q/k/v words, then [n_heads][chunks][head_dim + 2]
    // chunk partials (sum, max, denominator)
    unsigned long long *words;
    unsigned *err;                 // counts attention blocks whose poll gave up
    const StepState *st;
    int layer;
    // attention blocks per q head: at most step_qkv_attn_chunks(max_len) (0
    // there: at most kStepQkvAttnMaxChunks and kStepQkvAttnMaxBlocks in all),
    // and they must cover the step's context (chunks x 64 f32 / 128 bf16
    // positions); a launch of fewer than max_len needs serves short contexts
    // of a large state
    int chunks;
};

// Most attention blocks per q head, and per launch, in launch_step_qkv_attn.
constexpr int kStepQkvAttnMaxChunks = 32;
constexpr int kStepQkvAttnMaxBlocks = 512;
// Added to the error counter (StepQkvAttnArgs::err) by a chunked launch
// whose chunks do not cover the step's context, beside the count of
// attention blocks whose poll gave up.
constexpr unsigned kStepReachError = 1u << 20;

// Attention blocks per q head that launch_step_qkv_attn uses for caches of
// max_len positions (one per register pass of rows: 64 f32 or 128 bf16
// positions), or 0 when that is more than kStepQkvAttnMaxChunks or the
// launch's attention blocks more than kStepQkvAttnMaxBlocks.
int step_qkv_attn_chunks(size_t max_len, int kv_bf16, int n_heads);
// Cached positions one attention block of launch_step_qkv_attn takes (64 f32
// or 128 bf16).
int step_qkv_attn_rows(int kv_bf16);

// Exchange words launch_step_qkv_attn needs.
size_t step_qkv_attn_words(int q_rows, int kv_rows, int n_heads, int chunks);

// The attention blocks of launch_step_qkv_attn read cached rows in passes of
// up to this many positions without clamping to the context: the caches'
// allocation must extend this many rows (of head_dim f32) past the last head.
constexpr int kStepKvTailRows = 128;

bool step_qkv_attn_supported(int hidden, int n_heads, int n_kv_heads);
hipError_t launch_step_qkv_attn(hipStream_t s, const StepQkvAttnArgs &a);

// The q/k/v GEMV and the split attention of launch_step_attention in one
// launch (the same shapes as launch_step_qkv_attn take, any context): the
// GEMV blocks publish the rows as epoch words, then one block per (KV head,
// split of a.at.nsplit) requests its first cached rows, polls the words and
// attends, leaving the split partials (a.at.part_acc / part_ml) for
// launch_attn_combine, or the output with one split. a.chunks is unused.
hipError_t launch_step_qkv_stream(hipStream_t s, const StepQkvAttnArgs &a);

__device__ __forceinline__ void kv_load8(const float *p, float f[8]) {
    const float4 a = reinterpret_cast<const float4 *>(p)[0], b = reinterpret_cast<const float4 *>(p)[1];
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}
__device__ __forceinline__ void kv_load8(const uint16_t *p, float f[8]) {
    unpack8(*reinterpret_cast<const uint4 *>(p), f);
}
__device__ __forceinline__ float kv_load1(const float *p) { return *p; }
__device__ __forceinline__ float kv_load1(const uint16_t *p) { return bf16_to_f32(*p); }

}  // namespace th
