// The persistent decode kernel: the whole greedy decode loop of a Qwen3-style
// model (every layer of every step, the output projection and the greedy
// pick) in one cooperative launch.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "fused.h"

namespace th {

// Per-layer weights (bf16, row-major [out, in]) as the model uploaded them.
struct LayerWeights {
    const uint16_t *attn_norm, *q, *k, *v, *o, *q_norm, *k_norm, *mlp_norm, *gate, *up, *down;
};

// Replicas of every exchanged vector (one per XCD, so that pollers spread
// over distinct lines).
constexpr int kReplicas = 8;

struct DecodeParams {
    const LayerWeights *layers;  // device array [n_layers]
    const uint16_t *embed;       // [vocab][hidden]
    const uint16_t *norm;        // [hidden]
    const uint16_t *lm_head;     // [vocab][hidden] (the embedding table when tied)
    const float *rope;           // [max_len][head_dim/2][cos, sin]
    void *kv;                    // [layer][k|v][kv_head][max_len][head_dim]
    int kv_bf16;
    float *logits;               // [vocab]: the last step's logits
    StepState *step;             // pos, step, token on entry; updated on exit
    // Exchange buffers of (f32 bits | epoch << 32) words.
    unsigned long long *xchg_x;    // [kReplicas][hidden]
    unsigned long long *xchg_qkv;  // [q_dim + 2 kv_dim]
    unsigned long long *xchg_att;  // [kReplicas][q_dim]
    unsigned long long *xchg_h;    // [kReplicas][intermediate]
    unsigned long long *xchg_am;   // [kReplicas][2 * blocks]
    float *att_part;               // attention partials [kv_heads * group][splits][head_dim + 2]
    unsigned *att_count;           // [layers][kv_heads] arrival counters
    unsigned *status;              // [0]: abort flag / timeouts, [1]: protocol errors
    unsigned epoch_base;
    int steps;
    int hidden, intermediate, n_layers, n_heads, n_kv_heads, head_dim, vocab;
    int max_len, chunk, n_splits;  // attention: positions per split, splits
    float eps;
    long long timeout_ticks;       // bound on any single wait, in s_memrealtime ticks (100 MHz)
    // Optional trace of block 0 (null: off): [0] kernel start, then per traced
    // step and phase (5 per layer, then output projection and pick) four ticks:
    // its input arrived, its staged data was ready, it computed, it published
    // (0 where a phase has no such point). Low 32 bits of the 100 MHz clock.
    unsigned long long *trace;
    int trace_steps;
};

// Trace words a decode of `steps` traced steps writes.
__host__ __device__ inline size_t decode_trace_words(int n_layers, int steps) {
    return 1 + (size_t)steps * (size_t)(n_layers * 5 + 2) * 4;
}

// Epochs one decode step consumes (5 phases per layer, then lm_head and pick).
__host__ __device__ inline unsigned decode_epochs_per_step(int n_layers) { return (unsigned)(n_layers * 5 + 2); }

// Whether the persistent kernel supports this shape.
bool decode_supported(int hidden, int intermediate, int n_heads, int n_kv_heads, int head_dim, int vocab,
                      int blocks);

// Blocks the kernel runs with (one per CU).
int decode_blocks(int device);

hipError_t launch_decode(hipStream_t s, const DecodeParams &p, int blocks);

}  // namespace th
