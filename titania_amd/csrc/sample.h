// On-device sampling of the next token (model/sampler.rs:21-59).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "fused.h"

namespace th {

// Largest top_k sampled on the device, and largest vocabulary.
constexpr int kSampleMaxTopK = 256;
constexpr size_t kSampleMaxVocab = 32 * 8192;

// The sampler's parameters and generator state, in device memory.
struct SampleState {
    uint64_t rng;       // xorshift64* state (model/sampler.rs:62-76)
    uint64_t rng_prev;  // its value before the last draw
    float temperature;  // > 0
    float top_p;
    int top_k;          // in [1, min(vocab, kSampleMaxTopK)]
    uint32_t token;     // the draw, when no StepState records it
};

// Device scratch the sampler needs for a vocabulary (candidate keys).
size_t sample_scratch_bytes(size_t vocab);

// Draws a token from `logits`: into st (recorded like launch_pick, with the
// embedding row written for the next step) when st is not null, else into
// ss->token. Advances ss->rng by one draw.
hipError_t launch_sample(hipStream_t s, const float *logits, size_t vocab, void *scratch, SampleState *ss,
                         StepState *st, int advance, const PickEmbed &emb = PickEmbed());

}  // namespace th
