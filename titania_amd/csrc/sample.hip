// On-device sampling of the next token (model/sampler.rs:21-59): the top_k
// largest logits under total order (equal logits: the lower token first, an
// order the reference leaves unspecified), a softmax at the temperature over
// them, the shortest prefix whose probability reaches top_p, and a draw from
// that prefix with xorshift64*.
//
// Two launches: blocks of 8192 logits each sort their (key, inverted index)
// words in LDS and keep the largest kSampleMaxTopK; one block sorts those
// candidates and one thread then does the reference's arithmetic in its
// order (the softmax sum and the cumulative mass are sequential f32 folds).
#include "common.h"
#include "device_util.h"
#include "sample.h"

namespace th {

namespace {

constexpr int kSortThreads = 1024;
constexpr int kSortKeys = 8192;  // 64 KiB of LDS

// Bitonic sort of the block's kSortKeys words into descending order.
__device__ __forceinline__ void sort_desc(uint64_t *keys) {
    for (int size = 2; size <= kSortKeys; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int t = threadIdx.x; t < kSortKeys / 2; t += kSortThreads) {
                const int i = 2 * t - (t & (stride - 1)), j = i + stride;
                const uint64_t a = keys[i], b = keys[j];
                if ((a < b) == ((i & size) == 0)) {
                    keys[i] = b;
                    keys[j] = a;
                }
            }
            __syncthreads();
        }
    }
}

// The block's kSampleMaxTopK largest words, in order, to cand[block].
__global__ __launch_bounds__(kSortThreads) void topk_blocks_kernel(const float *__restrict__ logits, size_t vocab,
                                                                  uint64_t *__restrict__ cand) {
    __shared__ uint64_t keys[kSortKeys];
    const size_t base = (size_t)blockIdx.x * kSortKeys;
    for (int i = threadIdx.x; i < kSortKeys; i += kSortThreads) {
        const size_t t = base + i;
        keys[i] = t < vocab ? argmax_pack(logits[t], (uint32_t)t) : 0;  // real words are never 0
    }
    __syncthreads();
    sort_desc(keys);
    for (int i = threadIdx.x; i < kSampleMaxTopK; i += kSortThreads)
        cand[(size_t)blockIdx.x * kSampleMaxTopK + i] = keys[i];
}

// model/sampler.rs:66-76.
__device__ __forceinline__ uint64_t rng_next_u64(uint64_t &x) {
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    return x * 0x2545F4914F6CDD1DULL;
}

__device__ __forceinline__ float rng_next_f32(uint64_t &x) {
    return (float)(rng_next_u64(x) >> 40) / (float)(1u << 24);
}

__global__ __launch_bounds__(kSortThreads) void sample_kernel(const float *__restrict__ logits,
                                                             const uint64_t *__restrict__ cand, int n_cand,
                                                             SampleState *ss, StepState *st, int advance,
                                                             PickEmbed emb) {
    __shared__ uint64_t keys[kSortKeys];
    __shared__ float probs[kSampleMaxTopK];
    __shared__ uint32_t picked;
    for (int i = threadIdx.x; i < kSortKeys; i += kSortThreads) keys[i] = i < n_cand ? cand[i] : 0;
    __syncthreads();
    sort_desc(keys);
    if (threadIdx.x == 0) {
        // model/sampler.rs:35-58, in its order.
        const int k = ss->top_k;
        const float t = ss->temperature, top_p = ss->top_p;
        const float max = logits[argmax_index(keys[0])];
        for (int i = 0; i < k; ++i) probs[i] = expf((logits[argmax_index(keys[i])] - max) / t);
        float sum = 0.f;
        for (int i = 0; i < k; ++i) sum += probs[i];
        float cumulative = 0.f;
        int n = 0;
        for (int i = 0; i < k; ++i) {
            probs[i] /= sum;
            if (cumulative < top_p) {
                cumulative += probs[i];
                n += 1;
            }
        }
        // Steps after a stop token draw nothing (their picks are dropped).
        const bool draw = !(st && st->stopped);
        uint64_t x = ss->rng;
        if (draw) ss->rng_prev = x;
        float r = rng_next_f32(x) * cumulative;
        if (draw) ss->rng = x;
        uint32_t tok = argmax_index(keys[n - 1]);
        for (int i = 0; i < n; ++i) {
            r -= probs[i];
            if (r <= 0.f) {
                tok = argmax_index(keys[i]);
                break;
            }
        }
        if (st) tok = step_record(st, advance, tok);
        else ss->token = tok;
        picked = tok;
    }
    if (!st || !emb.table) return;
    __syncthreads();
    write_embedding(emb, picked);
}

}  // namespace

size_t sample_scratch_bytes(size_t vocab) {
    return (vocab + kSortKeys - 1) / kSortKeys * kSampleMaxTopK * sizeof(uint64_t);
}

hipError_t launch_sample(hipStream_t s, const float *logits, size_t vocab, void *scratch, SampleState *ss,
                         StepState *st, int advance, const PickEmbed &emb) {
    if (vocab == 0 || vocab > kSampleMaxVocab || (emb.table && emb.dim % 8)) return hipErrorInvalidValue;
    const unsigned blocks = (unsigned)((vocab + kSortKeys - 1) / kSortKeys);
    uint64_t *cand = static_cast<uint64_t *>(scratch);
    topk_blocks_kernel<<<blocks, kSortThreads, 0, s>>>(logits, vocab, cand);
    sample_kernel<<<1, kSortThreads, 0, s>>>(logits, cand, (int)(blocks * kSampleMaxTopK), ss, st, advance, emb);
    return hipGetLastError();
}

}  // namespace th
