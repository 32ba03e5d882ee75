// The XCD-parallel decode kernel: the whole greedy decode loop of a Qwen3-style
// model in one cooperative launch, laid out over the MI355X's eight XCDs the
// way tensor parallelism lays a layer out over eight devices.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "decode.h"
#include "fused.h"

namespace th {

constexpr int kXcds = 8;          // XCDs of an MI355X; KV head g lives on XCD g
constexpr int kXBlocksPerXcd = 32;

struct XDecodeParams {
    const LayerWeights *layers;  // device array [n_layers]
    const uint16_t *embed;       // [vocab][hidden]
    const uint16_t *norm;        // [hidden]
    const uint16_t *lm_head;     // [vocab][hidden] (the embedding table when tied)
    const float *rope;           // [max_len][head_dim/2][cos, sin]
    void *kv;                    // [layer][k|v][kv_head][max_len][head_dim]
    int kv_bf16;
    float *logits;               // [vocab]: the last step's logits
    StepState *step;
    // Exchange words (f32 bits | epoch << 32). *_loc are read only inside the
    // XCD that writes them (through its L2); part and am cross XCDs.
    unsigned long long *x_loc;    // [kXcds][hidden]
    unsigned long long *qkv_loc;  // [kXcds][(group + 2) * head_dim]
    unsigned long long *att_loc;  // [kXcds][kXBlocksPerXcd][group * (head_dim + 2)]
    unsigned long long *h_loc;    // [kXcds][intermediate / kXcds]
    unsigned long long *part;     // [2][kXcds][hidden]: o and down partial sums
    unsigned long long *am;       // [blocks][2]: per-block argmax (key, inverted index)
    unsigned *status;             // [0]: aborts / timeouts, [1]: protocol errors, [2]: XCD layout errors
    unsigned epoch_base;
    int steps;
    int hidden, intermediate, n_layers, n_heads, n_kv_heads, head_dim, vocab, max_len;
    float eps;
    long long timeout_ticks;       // bound on any single wait (100 MHz ticks)
    unsigned long long *trace;     // optional; the same layout as DecodeParams::trace
    int trace_steps;
};

// Epochs one decode step consumes.
__host__ __device__ inline unsigned xdecode_epochs_per_step(int n_layers) { return (unsigned)(n_layers * 7 + 1); }

// Whether the kernel supports this shape on a device with `blocks` CUs.
bool xdecode_supported(int hidden, int intermediate, int n_heads, int n_kv_heads, int head_dim, int vocab, int blocks);

hipError_t launch_xdecode(hipStream_t s, const XDecodeParams &p, int blocks);

}  // namespace th
