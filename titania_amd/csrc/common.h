// Internal definitions shared by the HIP device's translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>

#include "../../include/titania_hip.h"

// Concrete types behind the opaque handles of the C ABI.
struct th_device {
    int ordinal = 0;
    hipStream_t stream = nullptr;
    int num_cus = 0;
    // Device staging for token ids handed over from the host.
    uint32_t *tokens = nullptr;
    size_t tokens_cap = 0;
    // Scratch for partial results (attention splits, argmax partials). Grows on
    // demand outside graph capture.
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
    // The device address of the no-alloc entry points' fixed array (looked up
    // once, at th_device_create, with this device current).
    void *noalloc_scratch = nullptr;
    // One u32 the argmax kernels leave their result in.
    uint32_t *token_out = nullptr;
    // th_timer_begin / th_timer_end.
    hipEvent_t ev_begin = nullptr, ev_end = nullptr;
    // Between th_graph_begin and th_graph_end: the stream is being captured.
    bool capturing = false;
};

// A model takes ownership of weight handles it frees on destruction (the
// handles th_model_load uploads); null entries are skipped.
void th_model_own_weights(th_model *m, th_weight *const *w, size_t n);

struct th_buffer {
    float *ptr = nullptr;
    size_t len = 0;  // current length
    size_t cap = 0;  // length it was allocated with
};

struct th_weight {
    uint16_t *ptr = nullptr;  // bf16 bits, row-major
    size_t ndim = 0;
    size_t shape[2] = {0, 0};
    size_t numel = 0;
};

namespace th {

// Records a printf-style message as the calling thread's last error and returns `code`.
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Makes sure the device scratch holds at least `bytes`; returns its pointer or null.
void *scratch(th_device *dev, size_t bytes);

// The fixed array of the no-alloc entry points: its size, and its address on
// the current device.
size_t noalloc_scratch_bytes();
int noalloc_scratch_address(void **ptr);

}  // namespace th

#define TH_HIP(call)                                                                            \
    do {                                                                                        \
        hipError_t th_e_ = (call);                                                              \
        if (th_e_ != hipSuccess)                                                                \
            return th::fail(TH_ERR_HIP, "%s failed: %s (%s:%d)", #call, hipGetErrorString(th_e_), \
                            __FILE__, __LINE__);                                                \
    } while (0)

#define TH_REQUIRE(cond, ...)                                  \
    do {                                                       \
        if (!(cond)) return th::fail(TH_ERR_INVALID, __VA_ARGS__); \
    } while (0)

// Calls that allocate, move data to or from the host or wait are refused while
// the device's stream is being captured (th_graph_begin .. th_graph_end).
#define TH_NOT_CAPTURING(dev, what)                                                                        \
    TH_REQUIRE(!(dev)->capturing, "%s cannot run while the device's stream is being captured (th_graph_begin)", \
               what)

// Returns the status of `call` from the enclosing function unless it is TH_OK.
#define TRY(call)                 \
    do {                          \
        int rc_ = (call);         \
        if (rc_ != TH_OK) return rc_; \
    } while (0)

// Kernel launchers (host functions defined next to their kernels). Each queues
// work on `s` and returns the launch status; argument checks happen in the ABI layer.
namespace th {

hipError_t launch_embed(hipStream_t s, float *out, const uint16_t *table, size_t dim, const uint32_t *tokens,
                        size_t n);
hipError_t launch_copy(hipStream_t s, float *dst, const float *src, size_t len);
hipError_t launch_add(hipStream_t s, float *x, const float *y, size_t len);
hipError_t launch_silu_mul(hipStream_t s, float *gate, const float *up, size_t len);
// silu(gate) * up as split_bf16 terms hi/lo (len a multiple of 4).
hipError_t launch_silu_mul_split(hipStream_t s, const float *gate, const float *up, size_t len, uint16_t *hi,
                                 uint16_t *lo);
hipError_t launch_rmsnorm(hipStream_t s, float *x, size_t rows, const uint16_t *w, size_t dim, float eps);
// xb = rmsnorm(x (+)= y): if y, x += y first; xb may equal x.
hipError_t launch_add_rmsnorm(hipStream_t s, float *x, const float *y, float *xb, size_t rows,
                              const uint16_t *w, size_t dim, float eps);
// The same with the residual summed from ny partials y[z * y_stride] (z in
// order; ny = 0: none), the normalized rows to xb (f32) and/or to hi/lo as
// split_bf16 terms (either may be null, not both).
hipError_t launch_add_rmsnorm_parts(hipStream_t s, float *x, const float *y, int ny, size_t y_stride, float *xb,
                                    uint16_t *hi, uint16_t *lo, size_t rows, const uint16_t *w, size_t dim,
                                    float eps);
hipError_t launch_rope(hipStream_t s, float *x, size_t n, const float *table, size_t pos, size_t n_heads,
                       size_t head_dim);
// Two-pass argmax: partials need argmax_partials(n) u64 of scratch.
size_t argmax_partials(size_t n);
hipError_t launch_argmax(hipStream_t s, const float *x, size_t n, uint64_t *partials, uint32_t *token);
hipError_t launch_argmax_partials(hipStream_t s, const float *x, size_t n, uint64_t *partials);

// out[t*rows + r] = dot(w[r], x[t]) for t < n.
hipError_t launch_matmul(hipStream_t s, float *out, const uint16_t *w, size_t rows, size_t cols, const float *x,
                         size_t n);

// Attention over caches addressed as base + pos * pos_stride + head * head_stride
// (elements), f32 or bf16. The position is *pos_dev when pos_dev is not null.
struct AttnKernelArgs {
    float *out;
    const float *q;
    const void *k;
    const void *v;
    int n_heads, n_kv_heads, group;
    long long pos;
    const long long *pos_dev;
    long long pos_stride, head_stride;
    int nsplit;
    int kv_bf16;
    float scale;
    float *part_acc;  // [n][n_heads][nsplit][head_dim] when nsplit > 1
    float *part_ml;   // [n][n_heads][nsplit][2]
    // When set, the output goes here as split_bf16 terms [n][n_heads * head_dim]
    // (the o projection's GEMM input); `out` may then be scratch.
    uint16_t *out_hi, *out_lo;
};
// Splits of the sequence for n tokens (of head_dim) whose contexts reach at
// most max_len.
int attention_splits(size_t n, size_t n_heads, size_t n_kv_heads, size_t max_len, size_t head_dim);
// Scratch floats the partials of `nsplit` splits take (0 for one split).
size_t attention_scratch(size_t n, size_t n_heads, size_t head_dim, int nsplit);
hipError_t launch_attention(hipStream_t s, const AttnKernelArgs &k, size_t n, size_t head_dim);
// Prefill attention of an f32 cache through bf16 hi/lo planes of the keys and
// values: launch_attention's result, bit for bit, with each key and value
// split once per call instead of once per token tile. `planes` holds
// attention_planes_bytes(max_len, n_kv_heads) bytes of scratch (max_len: the
// positions the caches hold). Host positions only (no pos_dev).
size_t attention_planes_bytes(size_t max_len, size_t n_kv_heads);
bool attention_planes_supported(const AttnKernelArgs &k, size_t n, size_t head_dim);
// With split_kv false the planes already hold positions [0, pos + n): the
// q/k/v GEMM's epilogue wrote the new keys and values (QkvPostArgs::kh ..),
// and launch_kv_planes the earlier ones, before that GEMM.
hipError_t launch_attention_planes(hipStream_t s, const AttnKernelArgs &k, size_t n, size_t head_dim, void *planes,
                                   size_t planes_bytes, size_t max_len, bool split_kv = true);
// The planes of positions [0, valid) from the caches of k (the 64-position
// tile that holds `valid` gets zeros past it).
hipError_t launch_kv_planes(hipStream_t s, const AttnKernelArgs &k, size_t valid, void *planes, size_t planes_bytes,
                            size_t max_len);
// The four planes inside `planes` for caches of max_len positions.
struct PlanePtrs {
    uint16_t *kh, *kl, *vh, *vl;
    long long plane_len;
};
PlanePtrs attention_planes_of(void *planes, size_t max_len, size_t n_kv_heads);
// Merges attention partials of `heads` (token, head) pairs into out (f32) or,
// when hi is set, into hi/lo as split_bf16 terms.
hipError_t launch_attn_combine(hipStream_t s, float *out, const float *part_acc, const float *part_ml, size_t heads,
                               int nsplit, int hd, uint16_t *hi = nullptr, uint16_t *lo = nullptr);

}  // namespace th
