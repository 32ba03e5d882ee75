/*
 * titania_hip.h: the C ABI of the `hip` device, a gfx950 (MI355X) backend for
 * Titania's Qwen3 forward pass.
 *
 * The boundary replaced is the Rust trait `Device` (model/device.rs:9-89): one
 * entry point per trait method, with opaque handles for the associated types
 * `Buffer` (f32 activations) and `Weight` (bf16 tensor). Each declaration cites
 * the trait method it stands for. Where the trait panics on misuse (the length
 * asserts of model/cpu.rs:22,40,52-53 and model/titania.rs:125,140,147,156-157,188)
 * these functions return TH_ERR_INVALID before touching the GPU, and
 * th_last_error() says why.
 *
 * Beyond the trait, the device offers fused operations whose results equal the
 * composition of the primitives in the order model/model.rs:93-149 calls them,
 * and the forward pass itself (model/model.rs:83-149) with a device-resident
 * greedy decode loop.
 *
 * Threading: a device and its handles belong to one host thread at a time
 * (the reference builds and uses its model on one worker thread,
 * cli/run.rs:49,121-127). All work runs in order on one HIP stream per device.
 */
#ifndef TITANIA_HIP_H
#define TITANIA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define TH_API __attribute__((visibility("default")))
#else
#define TH_API
#endif

/* Status codes. */
#define TH_OK 0
#define TH_ERR_INVALID 1 /* misuse: a length, shape, offset or position out of range */
#define TH_ERR_HIP 2     /* a HIP runtime call failed */
#define TH_ERR_NOMEM 3   /* device or host allocation failed */

typedef struct th_device th_device; /* a GPU, its stream and its scratch memory */
typedef struct th_buffer th_buffer; /* model/device.rs:10-13 `Device::Buffer` */
typedef struct th_weight th_weight; /* model/device.rs:14-15 `Device::Weight` */

/* Message describing the last failure on the calling thread ("" if none). */
TH_API const char *th_last_error(void);

/* Opens GPU `ordinal` (stands in for `Cpu` / `Titania::new`, cli/run.rs:121-128). */
TH_API int th_device_create(int ordinal, th_device **out);
TH_API void th_device_destroy(th_device *dev);
/* Waits for all work queued on the device. */
TH_API int th_device_synchronize(th_device *dev);

/* model/device.rs:17-18 `upload`: copies a row-major bf16 tensor (raw bits,
 * model/weights.rs:13-17) of `ndim` (1 or 2) dimensions into device memory. */
TH_API int th_upload(th_device *dev, const uint16_t *data, const size_t *shape, size_t ndim, th_weight **out);
TH_API void th_weight_free(th_device *dev, th_weight *w);
/* Shape of a weight: writes ndim and up to 2 extents. */
TH_API int th_weight_shape(const th_weight *w, size_t *shape, size_t *ndim);

/* model/device.rs:20-21 `alloc`: a zeroed buffer of `len` f32 activations. */
TH_API int th_alloc(th_device *dev, size_t len, th_buffer **out);
TH_API void th_buffer_free(th_device *dev, th_buffer *buf);
/* model/device.rs:23-26 `resize`: len <= the allocated length; contents gained are undefined. */
TH_API int th_resize(th_device *dev, th_buffer *buf, size_t len);
TH_API size_t th_buffer_len(const th_buffer *buf);
/* model/device.rs:28-29 `read`: copies the buffer's `len` activations out (blocking). */
TH_API int th_read(th_device *dev, const th_buffer *buf, float *out, size_t len);
/* model/device.rs:31-32 `write`: `len` must equal the buffer's length. */
TH_API int th_write(th_device *dev, th_buffer *buf, const float *data, size_t len);
/* model/device.rs:34-42 `copy`: dst[dst_offset..][..len] = src[src_offset..][..len]. */
TH_API int th_copy(th_device *dev, th_buffer *dst, size_t dst_offset, const th_buffer *src, size_t src_offset,
            size_t len);

/* model/device.rs:44-46 `embed`: out[t] = table[tokens[t]]; out.len == n * table.shape[1]. */
TH_API int th_embed(th_device *dev, th_buffer *out, const th_weight *table, const uint32_t *tokens, size_t n);
/* model/device.rs:48-51 `matmul`: out[t] = w . x[t] for w [rows, cols]; n = x.len / cols. */
TH_API int th_matmul(th_device *dev, th_buffer *out, const th_weight *w, const th_buffer *x);
/* model/device.rs:53-54 `add`: x += y. */
TH_API int th_add(th_device *dev, th_buffer *x, const th_buffer *y);
/* model/device.rs:56-58 `rmsnorm`: each weight.len-long row of x. */
TH_API int th_rmsnorm(th_device *dev, th_buffer *x, const th_weight *weight, float eps);
/* model/device.rs:60-66 `rope`: table[(p * head_dim/2 + i) * 2..][..2] = (cos, sin). */
TH_API int th_rope(th_device *dev, th_buffer *x, const th_buffer *table, size_t pos, size_t n_heads, size_t head_dim);
/* model/device.rs:68-85 `attention`: caches laid out [position][n_kv_heads][head_dim]. */
TH_API int th_attention(th_device *dev, th_buffer *out, const th_buffer *q, const th_buffer *k_cache,
                 const th_buffer *v_cache, size_t pos, size_t n_heads, size_t head_dim, size_t n_kv_heads);
/* th_attention without any allocation: its split partials go to a fixed
 * 16 MiB array that the library holds on each GPU until the process ends, so
 * that callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc) can call it. No counterpart
 * in model/device.rs. Same arguments, checks and results as th_attention; a
 * call whose partials need more than 16 MiB (n * n_heads * splits *
 * (head_dim + 2) floats, at most 256 splits for one token: one token of up to
 * 126 heads of head_dim 128 at any context fits, a 2048-token prompt of 32
 * heads at 8192 positions does not) returns TH_ERR_INVALID. Every call on a GPU
 * shares that GPU's array: calls that overlap on one GPU (two device handles of one GPU, two
 * threads) race. */
TH_API int th_attention_noalloc(th_device *dev, th_buffer *out, const th_buffer *q, const th_buffer *k_cache,
                                const th_buffer *v_cache, size_t pos, size_t n_heads, size_t head_dim,
                                size_t n_kv_heads);
/* model/device.rs:87-88 `silu_mul`: gate = silu(gate) * up. */
TH_API int th_silu_mul(th_device *dev, th_buffer *gate, const th_buffer *up);

/* Device-side timing: th_timer_begin records an event on the device's stream,
 * th_timer_end records another, waits for it and gives the milliseconds between
 * the two (the GPU time of the work queued in between). */
TH_API int th_timer_begin(th_device *dev);
TH_API int th_timer_end(th_device *dev, float *ms);

/* HIP graphs of the device's stream, for launch-bound sequences of calls (no
 * counterpart in model/device.rs; the graph_begin / graph_end / graph_launch
 * extension of the Device boundary). th_graph_begin starts capturing the
 * stream in thread-local mode: the compute calls that follow (copy, matmul of
 * fewer than 16 tokens, add, rmsnorm, rope, attention, silu_mul, the fused
 * extensions) are recorded, not run. th_graph_end stops the capture and
 * instantiates it; th_graph_launch queues one replay on the stream, reading
 * and writing the buffers named at capture time. While capturing, the calls
 * that allocate, move data to or from the host, wait or free (upload, alloc,
 * read, write, embed, argmax, sample, the timer, synchronize, the frees and
 * destroys, the model and state calls, a matmul of 16 or more tokens, and an
 * attention whose partials outgrow the device's scratch) return
 * TH_ERR_INVALID (the frees leave their handle valid); the capture stays open
 * until th_graph_end. th_device_destroy discards an open capture. */
typedef struct th_graph th_graph;
TH_API int th_graph_begin(th_device *dev);
TH_API int th_graph_end(th_device *dev, th_graph **out);
TH_API int th_graph_launch(th_device *dev, const th_graph *graph);
TH_API void th_graph_free(th_device *dev, th_graph *graph);

/* ---- fused extensions (each equals its composition of trait methods) ---- */

/* x += y, then xb = rmsnorm(x) with `weight` (the add, copy and rmsnorm of
 * model/model.rs:132-136). y may be NULL for copy + rmsnorm alone (model.rs:106-107),
 * and may be xb itself (the residual add of a projection written to xb, then
 * the norm into xb). Default methods `add_rmsnorm` / `copy_rmsnorm` of the
 * trait extension (titania_amd/rust/patches/model-device.rs.patch). */
TH_API int th_add_rmsnorm(th_device *dev, th_buffer *x, const th_buffer *y, th_buffer *xb, const th_weight *weight,
                   float eps);
/* The attention block's input side for n = xb.len / hidden tokens at
 * positions pos.. (model/model.rs:108-120 in one call): q, k, v = wq, wk, wv
 * . xb; q and k RMSNorm'd per head by q_norm / k_norm (either may be NULL) and
 * rotated with the rope table; k and v copied into the caches, laid out
 * [position][n_kv_heads][head_dim] as th_attention reads them, at pos. Equals
 * matmul x 3, rmsnorm x 2, rope x 2 and copy x 2 in that order within
 * rounding; afterwards k and v hold the projections before the norm and
 * rotation (nothing reads them after the copies). Default method
 * `qkv_rope_append` of the trait extension. */
TH_API int th_qkv_rope_append(th_device *dev, th_buffer *q, th_buffer *k, th_buffer *v, const th_weight *wq,
                              const th_weight *wk, const th_weight *wv, const th_weight *q_norm,
                              const th_weight *k_norm, const th_buffer *xb, const th_buffer *rope,
                              th_buffer *k_cache, th_buffer *v_cache, size_t pos, size_t n_heads, size_t n_kv_heads,
                              size_t head_dim, float eps);
/* gate = silu(w_gate . xb) * (w_up . xb) (model/model.rs:137-139: matmul,
 * matmul, silu_mul); `up` is scratch, its contents afterwards unspecified.
 * Default method `gate_up_silu` of the trait extension. */
TH_API int th_gate_up_silu(th_device *dev, th_buffer *gate, th_buffer *up, const th_weight *w_gate,
                           const th_weight *w_up, const th_buffer *xb);
/* Greedy choice (model/sampler.rs:21-33 at temperature 0): index of the largest
 * of the buffer's values under IEEE total order, lowest index on ties. */
TH_API int th_argmax(th_device *dev, const th_buffer *logits, uint32_t *token);
/* model/sampler.rs:21-59 `Sampler::sample` over a device buffer: the top_k
 * largest values (top_k clamped to [1, len], at most 256 on the device; len at
 * most 262144); at temperature 0 the largest, as th_argmax; otherwise a softmax
 * at the temperature over the top_k, the shortest prefix of them whose
 * probability reaches top_p, and a draw from that prefix with the xorshift64*
 * generator whose state is *rng (sampler.rs:62-76; Sampler::new seeds it with
 * max(seed, 1)); *rng advances by one draw. Equal values rank by lower index
 * (the reference leaves their order unspecified). At a nonzero temperature
 * top_p must be > 0 (the reference panics otherwise). */
TH_API int th_sample(th_device *dev, const th_buffer *logits, float temperature, size_t top_k, float top_p,
                     uint64_t *rng, uint32_t *token);

/* ---- the forward pass (model/model.rs) ---- */

/* Architecture (model/config.rs:9-36, head_dim resolved as config.rs:32-35 does). */
typedef struct th_config {
    int64_t hidden_size;
    int64_t intermediate_size;
    int64_t num_hidden_layers;
    int64_t num_attention_heads;
    int64_t num_key_value_heads;
    int64_t head_dim;
    int64_t vocab_size;
    float rms_norm_eps;
    float rope_theta;
    int64_t tie_word_embeddings;
} th_config;

typedef struct th_model th_model; /* model/model.rs:10-19 `Model` */
typedef struct th_state th_state; /* model/model.rs:152-172 `State` */

/* Builds a model from uploaded weights (model/model.rs:40-77). `weights` holds
 * 11 handles per layer in the order model.rs:50-60 loads them (input_layernorm,
 * q_proj, k_proj, v_proj, o_proj, q_norm, k_norm, post_attention_layernorm,
 * gate_proj, up_proj, down_proj; q_norm and k_norm may be NULL), then
 * embed_tokens, norm, and lm_head (NULL when tie_word_embeddings). The model
 * borrows the handles: free them only after th_model_destroy. */
TH_API int th_model_create(th_device *dev, const th_config *config, const th_weight *const *weights, size_t n_weights,
                    th_model **out);
TH_API void th_model_destroy(th_model *model);

/* model/config.rs:29-35 `Config::load`: the architecture from a Hugging Face
 * config.json as serde reads it (unsigned sizes from integer literals, the two
 * f32 fields from any number, head_dim absent or null -> hidden_size /
 * num_attention_heads, tie_word_embeddings absent -> false, other keys
 * ignored). Needs no GPU. */
TH_API int th_config_load(const char *path, th_config *out);
/* model/model.rs:40-77 `Model::load`: config.json and model.safetensors from
 * `dir` (model/weights.rs:19-81: every tensor BF16; q_norm / k_norm optional;
 * lm_head.weight only when not tied), uploaded to `dev`. Errors name the file,
 * or the tensor that is missing or not BF16. The model owns these weights and
 * frees them in th_model_destroy. */
TH_API int th_model_load(th_device *dev, const char *dir, th_model **out);
/* The architecture a model was built with. */
TH_API int th_model_config(const th_model *model, th_config *out);

#define TH_KV_F32 0  /* f32 caches, as the reference stores them (model/model.rs:206-207) */
#define TH_KV_BF16 1 /* bf16 caches: half the bytes per position */

/* model/model.rs:176-211 `State::new` for sequences of up to max_len tokens.
 * The caches are laid out per layer and per KV head: [layer][kv_head][max_len][head_dim].
 * Besides the caches, the first forward or decode allocates buffers for
 * prefill chunks of up to min(8192, max_len) tokens, kept for the state's
 * life: 4 * (3 hidden + 2 q + 2 kv + 2 intermediate) bytes a token of
 * activations plus the GEMM's split scratch, about 1.9 GB at the Qwen3-4B
 * shape once max_len >= 8192 (0.25 GB at max_len 1024). Size max_len to the
 * longest sequence the state will hold. */
TH_API int th_state_create(th_model *model, size_t max_len, int kv_dtype, th_state **out);
TH_API void th_state_destroy(th_state *state);

#define TH_PATH_OPS 0   /* one trait primitive per step, exactly as model.rs:103-148 calls them */
#define TH_PATH_FUSED 1 /* fused kernels, same results within rounding */
#define TH_PATH_TRAIT 2 /* the trait extension's methods in the order the patched forward_batch calls them
                           (titania_amd/rust/patches/model-model.rs.patch), on the caches of TH_PATH_OPS */

/* model/model.rs:83-91 `Model::forward`: runs n tokens, the first at position
 * pos, adds their keys and values to the caches and writes the logits of the
 * token after the last into `logits` (vocab_size floats; NULL to skip the copy). */
TH_API int th_forward(th_model *model, th_state *state, const uint32_t *tokens, size_t n, size_t pos, float *logits,
               int path);

/* Greedy decode as model/chat.rs:149-178 drives it at temperature 0, kept on
 * the device: `steps` times, pick the argmax of the current logits and feed it
 * at position pos, pos + 1, ... The first pick is from the logits the last
 * th_forward left. Writes the picked tokens to out_tokens and, if out_logits is
 * not NULL, the logits after each fed token (steps * vocab_size floats). One
 * step is one HIP graph replay; the host waits once, at the end. */
TH_API int th_decode(th_model *model, th_state *state, size_t pos, size_t steps, uint32_t *out_tokens, float *out_logits);

/* th_decode with every pick drawn as th_sample draws it (model/chat.rs:149-178
 * driving a Sampler from model/sampler.rs), kept on the device: *rng is the
 * generator state before the first draw and is left after the last. The
 * logits never leave the device. Temperature 0 is th_decode. */
TH_API int th_decode_sample(th_model *model, th_state *state, size_t pos, size_t steps, float temperature,
                            size_t top_k, float top_p, uint64_t *rng, uint32_t *out_tokens);

/* The reply loop of model/chat.rs:147-178 (`Chat::generate` once its prompt
 * has been fed), kept on the device: from the logits the last th_forward left,
 * pick (temperature 0) or draw (as th_decode_sample) a token; if it is one of
 * the n_stop (1..8) stop tokens, stop; else feed it at the next position (pos,
 * pos + 1, ...) and go on, for at most max_tokens tokens. Writes the tokens to
 * out_tokens (room for max_tokens) and their count to *n_out. When the last is
 * a stop token it was not fed, and the conversation has grown by *n_out - 1
 * tokens; otherwise by *n_out. The host looks for a stop every 8 steps (the
 * steps after it repeat the last fed token and change nothing). rng may be
 * NULL at temperature 0. No counterpart in the trait: the reference's Chat
 * drives Model::forward and Sampler::sample one token at a time. */
TH_API int th_generate(th_model *model, th_state *state, size_t pos, size_t max_tokens, const uint32_t *stop,
                       size_t n_stop, float temperature, size_t top_k, float top_p, uint64_t *rng,
                       uint32_t *out_tokens, size_t *n_out);

#ifdef __cplusplus
}
#endif

#endif /* TITANIA_HIP_H */
