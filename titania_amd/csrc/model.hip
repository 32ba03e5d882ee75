// The forward pass of model/model.rs on the hip device: Model (model.rs:10-35),
// State (model.rs:152-233), Model::forward (model.rs:83-149), and a greedy
// decode loop that stays on the device (model/chat.rs:149-178 at temperature 0).
//
// Three paths compute the same function:
//  - TH_PATH_OPS calls the trait's primitives through the public C ABI in
//    exactly the order model.rs:103-148 does, on the reference's state layout
//    (BATCH-token chunks, position-major f32 caches);
//  - TH_PATH_TRAIT calls the trait extension's fused methods where the
//    patched forward_batch calls them, on the same state;
//  - TH_PATH_FUSED runs the fused kernels on caches laid out per layer and per
//    KV head ([layer][k|v][kv_head][max_len][head_dim], f32 or bf16), and is
//    what a decode step captures into a HIP graph.
#include <cmath>
#include <cstring>
#include <new>
#include <vector>

#include <cstdlib>

#include "common.h"
#include "fused.h"
#include "gemm.h"
#include "sample.h"
#include "step.h"

namespace {

constexpr size_t kBatch = 64;          // model/model.rs:8 BATCH (the ops path)
// Tokens per chunk on the fused path. Larger chunks make larger GEMMs and
// fewer attention launches: an 8192-token prompt of the Qwen3-4B shape took
// 202.8 / 197.1 / 194.5 ms in chunks of 2048 / 4096 / 8192 (Qwen3-0.6B:
// 51.7 / 51.2 / 48.6 ms). A state holds the chunk's activations, GEMM
// scratch and attention partials, about 3 GB at the 4B shape.
constexpr size_t kFusedBatch = 8192;
constexpr size_t kWeightsPerLayer = 11;

struct Layer {
    const th_weight *attn_norm, *q, *k, *v, *o, *q_norm, *k_norm, *mlp_norm, *gate, *up, *down;
};

}  // namespace

struct th_model {
    th_device *dev = nullptr;
    th_config c{};
    std::vector<Layer> layers;
    const th_weight *embed = nullptr, *norm = nullptr, *lm_head = nullptr;
    const th_weight *out_proj() const { return lm_head ? lm_head : embed; }  // model.rs:147
    std::vector<th_weight *> owned;  // freed with the model (th_model_load)
};

void th_model_own_weights(th_model *m, th_weight *const *w, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (w[i]) m->owned.push_back(w[i]);
}

struct th_state {
    th_model *m = nullptr;
    size_t max_len = 0;
    int kv_dtype = TH_KV_F32;
    int path = -1;  // the path that has filled the caches (-1: none yet)

    // Shared by both paths.
    th_buffer *rope = nullptr;    // model.rs:192-194
    th_buffer *logits = nullptr;  // [vocab]

    // TH_PATH_OPS: the reference's State buffers (model.rs:181-207).
    th_buffer *x = nullptr, *xb = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *att = nullptr,
              *gate = nullptr, *up = nullptr;
    std::vector<th_buffer *> k_cache, v_cache;

    // TH_PATH_FUSED.
    size_t fb = 0;  // token capacity of the fused buffers
    float *fx = nullptr, *fxb = nullptr, *fq = nullptr, *fk = nullptr, *fv = nullptr, *fatt = nullptr,
          *fgate = nullptr, *fup = nullptr, *fy = nullptr;
    void *fsplit = nullptr;   // bf16 hi/lo halves of a GEMM input (fb tokens x fsplit_cols)
    size_t fsplit_cols = 0;
    size_t fsplit_bytes = 0;
    void *kv = nullptr;  // all caches, one allocation
    size_t kv_elem = 4;
    float *attn_part = nullptr;  // attention partials for the fused path
    size_t attn_part_floats = 0;
    void *kv_planes = nullptr;  // a layer's keys and values as bf16 hi/lo planes (f32 caches, prefill)
    size_t kv_planes_bytes = 0;
    uint64_t *argmax_part = nullptr;
    th::StepState *step = nullptr;  // device
    uint32_t *tokens_dev = nullptr;
    size_t tokens_dev_cap = 0;
    float *logits_dev = nullptr;  // decode logits kept for the caller
    size_t logits_dev_cap = 0;
    hipGraph_t graph = nullptr;  // one decode step
    hipGraphExec_t graph_exec = nullptr;
    hipGraph_t graph_n = nullptr;  // kGraphSteps decode steps
    hipGraphExec_t graph_n_exec = nullptr;
    // The same with the streaming attention, for states whose step takes the
    // chunked launch only while the context is short (step_dual).
    hipGraph_t graph_l = nullptr;
    hipGraphExec_t graph_l_exec = nullptr;
    hipGraph_t graph_ln = nullptr;
    hipGraphExec_t graph_ln_exec = nullptr;

    // The captured decode step's buffers (fixed addresses for the graph).
    bool step_fused = false;
    float *sx_a = nullptr, *sx_b = nullptr, *s_y = nullptr, *s_qkv = nullptr, *s_att = nullptr, *s_o = nullptr,
          *s_h = nullptr;
    uint64_t *s_part = nullptr;
    unsigned long long *s_words = nullptr;  // q/k/v words of the single-launch q/k/v + attention
    unsigned *s_err = nullptr;              // its attention blocks whose poll gave up
    uint32_t step_epoch = 0;                // StepState::epoch at the next decode call
    bool graph_keep = false;                // whether the captured step copies out the logits
    // Sampled decode (th_decode_sample): the sampler's device state and
    // candidate scratch; whether the step draws instead of picking the argmax.
    th::SampleState *s_sample = nullptr;
    void *s_cand = nullptr;
    bool sampling = false;
};

namespace {

using th::fail;

void free_dev(void *p) {
    if (p) (void)hipFree(p);
}

// model/model.rs:239-250: (cos, sin) of pos * theta^(-2i/head_dim), pushed as [cos, sin].
std::vector<float> rope_table(size_t max_len, size_t head_dim, float theta) {
    size_t half = head_dim / 2;
    std::vector<float> t;
    t.reserve(max_len * head_dim);
    for (size_t pos = 0; pos < max_len; ++pos) {
        for (size_t i = 0; i < half; ++i) {
            float freq = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
            float a = (float)pos * freq;
            t.push_back(cosf(a));
            t.push_back(sinf(a));
        }
    }
    return t;
}

int check_shape(const th_weight *w, size_t r, size_t c, const char *what, size_t layer) {
    if (!w) return fail(TH_ERR_INVALID, "layer %zu: missing %s", layer, what);
    if (c == 0) {
        if (w->numel != r) return fail(TH_ERR_INVALID, "layer %zu: %s has %zu elements, not %zu", layer, what, w->numel, r);
        return TH_OK;
    }
    if (w->ndim != 2 || w->shape[0] != r || w->shape[1] != c)
        return fail(TH_ERR_INVALID, "layer %zu: %s is not [%zu, %zu]", layer, what, r, c);
    return TH_OK;
}

// Device pointer of the cache of (layer, k or v) on the fused path.
void *cache_ptr(th_state *s, size_t layer, int which) {
    const th_config &c = s->m->c;
    size_t per = (size_t)c.num_key_value_heads * s->max_len * (size_t)c.head_dim;
    return static_cast<char *>(s->kv) + ((layer * 2 + which) * per) * s->kv_elem;
}

int ensure_ops_state(th_state *s) {
    if (s->x) return TH_OK;
    th_model *m = s->m;
    const th_config &c = m->c;
    size_t qd = (size_t)(c.num_attention_heads * c.head_dim), kvd = (size_t)(c.num_key_value_heads * c.head_dim);
    size_t widths[8] = {(size_t)c.hidden_size, (size_t)c.hidden_size, qd, kvd, kvd, qd, (size_t)c.intermediate_size,
                        (size_t)c.intermediate_size};
    th_buffer **bufs[8] = {&s->x, &s->xb, &s->q, &s->k, &s->v, &s->att, &s->gate, &s->up};
    for (int i = 0; i < 8; ++i) {
        int rc = th_alloc(m->dev, kBatch * widths[i], bufs[i]);
        if (rc) return rc;
    }
    for (int64_t l = 0; l < c.num_hidden_layers; ++l) {
        th_buffer *kb = nullptr, *vb = nullptr;
        int rc = th_alloc(m->dev, s->max_len * kvd, &kb);
        if (rc) return rc;
        s->k_cache.push_back(kb);
        rc = th_alloc(m->dev, s->max_len * kvd, &vb);
        if (rc) return rc;
        s->v_cache.push_back(vb);
    }
    return TH_OK;
}

// model/model.rs:93-149, one primitive per step, for n <= BATCH tokens.
int forward_batch_ops(th_state *s, const uint32_t *tokens, size_t n, size_t pos) {
    th_model *m = s->m;
    th_device *d = m->dev;
    const th_config &c = m->c;
    const float eps = c.rms_norm_eps;
    const size_t hd = (size_t)c.head_dim, H = (size_t)c.hidden_size;
    const size_t kv_dim = (size_t)c.num_key_value_heads * hd;
    size_t widths[8] = {H, H, (size_t)c.num_attention_heads * hd, kv_dim, kv_dim, (size_t)c.num_attention_heads * hd,
                        (size_t)c.intermediate_size, (size_t)c.intermediate_size};
    th_buffer *bufs[8] = {s->x, s->xb, s->q, s->k, s->v, s->att, s->gate, s->up};
    for (int i = 0; i < 8; ++i) TRY(th_resize(d, bufs[i], n * widths[i]));  // State::batch

    TRY(th_embed(d, s->x, m->embed, tokens, n));
    for (size_t i = 0; i < m->layers.size(); ++i) {
        const Layer &L = m->layers[i];
        TRY(th_copy(d, s->xb, 0, s->x, 0, n * H));
        TRY(th_rmsnorm(d, s->xb, L.attn_norm, eps));
        TRY(th_matmul(d, s->q, L.q, s->xb));
        TRY(th_matmul(d, s->k, L.k, s->xb));
        TRY(th_matmul(d, s->v, L.v, s->xb));
        if (L.q_norm) TRY(th_rmsnorm(d, s->q, L.q_norm, eps));
        if (L.k_norm) TRY(th_rmsnorm(d, s->k, L.k_norm, eps));
        TRY(th_rope(d, s->q, s->rope, pos, (size_t)c.num_attention_heads, hd));
        TRY(th_rope(d, s->k, s->rope, pos, (size_t)c.num_key_value_heads, hd));
        TRY(th_copy(d, s->k_cache[i], pos * kv_dim, s->k, 0, n * kv_dim));
        TRY(th_copy(d, s->v_cache[i], pos * kv_dim, s->v, 0, n * kv_dim));
        TRY(th_attention(d, s->att, s->q, s->k_cache[i], s->v_cache[i], pos, (size_t)c.num_attention_heads, hd,
                         (size_t)c.num_key_value_heads));
        TRY(th_matmul(d, s->xb, L.o, s->att));
        TRY(th_add(d, s->x, s->xb));

        TRY(th_copy(d, s->xb, 0, s->x, 0, n * H));
        TRY(th_rmsnorm(d, s->xb, L.mlp_norm, eps));
        TRY(th_matmul(d, s->gate, L.gate, s->xb));
        TRY(th_matmul(d, s->up, L.up, s->xb));
        TRY(th_silu_mul(d, s->gate, s->up));
        TRY(th_matmul(d, s->xb, L.down, s->gate));
        TRY(th_add(d, s->x, s->xb));
    }
    TRY(th_resize(d, s->xb, H));
    TRY(th_copy(d, s->xb, 0, s->x, (n - 1) * H, H));
    TRY(th_rmsnorm(d, s->xb, m->norm, eps));
    TRY(th_matmul(d, s->logits, m->out_proj(), s->xb));
    return TH_OK;
}

// The patched forward_batch (titania_amd/rust/patches/model-model.rs.patch)
// through the trait extension's methods, for n <= BATCH tokens, on the ops
// path's state: copy_rmsnorm / add_rmsnorm for the residual adds and norms,
// qkv_rope_append for model.rs:108-120, gate_up_silu for model.rs:137-139; the
// attention, the o and down projections and the final norm as the primitives.
int forward_batch_trait(th_state *s, const uint32_t *tokens, size_t n, size_t pos) {
    th_model *m = s->m;
    th_device *d = m->dev;
    const th_config &c = m->c;
    const float eps = c.rms_norm_eps;
    const size_t hd = (size_t)c.head_dim, H = (size_t)c.hidden_size;
    const size_t nh = (size_t)c.num_attention_heads, nkv = (size_t)c.num_key_value_heads;
    size_t widths[8] = {H, H, nh * hd, nkv * hd, nkv * hd, nh * hd, (size_t)c.intermediate_size,
                        (size_t)c.intermediate_size};
    th_buffer *bufs[8] = {s->x, s->xb, s->q, s->k, s->v, s->att, s->gate, s->up};
    for (int i = 0; i < 8; ++i) TRY(th_resize(d, bufs[i], n * widths[i]));  // State::batch

    TRY(th_embed(d, s->x, m->embed, tokens, n));
    for (size_t i = 0; i < m->layers.size(); ++i) {
        const Layer &L = m->layers[i];
        // The previous layer's down projection (in xb) added into x, then the
        // attention norm; the first layer only normalizes.
        TRY(th_add_rmsnorm(d, s->x, i ? s->xb : nullptr, s->xb, L.attn_norm, eps));
        TRY(th_qkv_rope_append(d, s->q, s->k, s->v, L.q, L.k, L.v, L.q_norm, L.k_norm, s->xb, s->rope, s->k_cache[i],
                               s->v_cache[i], pos, nh, nkv, hd, eps));
        TRY(th_attention(d, s->att, s->q, s->k_cache[i], s->v_cache[i], pos, nh, hd, nkv));
        TRY(th_matmul(d, s->xb, L.o, s->att));
        TRY(th_add_rmsnorm(d, s->x, s->xb, s->xb, L.mlp_norm, eps));
        TRY(th_gate_up_silu(d, s->gate, s->up, L.gate, L.up, s->xb));
        TRY(th_matmul(d, s->xb, L.down, s->gate));
    }
    if (!m->layers.empty()) TRY(th_add(d, s->x, s->xb));
    TRY(th_resize(d, s->xb, H));
    TRY(th_copy(d, s->xb, 0, s->x, (n - 1) * H, H));
    TRY(th_rmsnorm(d, s->xb, m->norm, eps));
    TRY(th_matmul(d, s->logits, m->out_proj(), s->xb));
    return TH_OK;
}

// Attention blocks per q head of this state's chunked q/k/v + attention
// launch: the chunks max_len needs, at most 16 and fewer than 512 blocks in
// all (the reach in which that launch beats the streaming one, below); 0
// where the launch does not serve the model.
int step_reach_chunks(const th_state *s) {
    const th_config &c = s->m->c;
    const int nh = (int)c.num_attention_heads, nkv = (int)c.num_key_value_heads;
    if (!th::step_qkv_attn_supported((int)c.hidden_size, nh, nkv) || s->m->layers.size() >= 64) return 0;
    const long long rows = th::step_qkv_attn_rows(s->kv_dtype == TH_KV_BF16);
    int k = (int)std::min<long long>(((long long)s->max_len + rows - 1) / rows, 16);
    while (k > 0 && k * nh >= th::kStepQkvAttnMaxBlocks) --k;
    return k;
}

int ensure_fused_state(th_state *s) {
    if (s->fx) return TH_OK;
    th_model *m = s->m;
    const th_config &c = m->c;
    const size_t H = (size_t)c.hidden_size, I = (size_t)c.intermediate_size, hd = (size_t)c.head_dim;
    const size_t qd = (size_t)c.num_attention_heads * hd, kvd = (size_t)c.num_key_value_heads * hd;
    s->fb = std::min(kFusedBatch, s->max_len);
    struct {
        float **p;
        size_t n;
    } bufs[] = {{&s->fx, H}, {&s->fxb, H}, {&s->fq, qd}, {&s->fk, kvd}, {&s->fv, kvd},
                {&s->fatt, qd}, {&s->fgate, I}, {&s->fup, I}, {&s->fy, H}};
    for (auto &b : bufs) TH_HIP(hipMalloc(b.p, s->fb * b.n * sizeof(float)));
    if (s->fb >= th::kGemmMinTokens) {
        s->fsplit_cols = std::max(std::max(H, qd), I);
        s->fsplit_bytes = th::gemm_scratch_bytes(s->fb, s->fsplit_cols, H);
        TH_HIP(hipMalloc(&s->fsplit, s->fsplit_bytes));
    }
    s->kv_elem = s->kv_dtype == TH_KV_BF16 ? 2 : 4;
    size_t kv_bytes = (size_t)c.num_hidden_layers * 2 * kvd * s->max_len * s->kv_elem;
    // Tail rows that the decode step's attention may read (and ignore) past
    // the last head's max_len positions.
    TH_HIP(hipMalloc(&s->kv, kv_bytes + (size_t)th::kStepKvTailRows * hd * sizeof(float)));
    // Attention partials: enough for any chunk of up to fb tokens at any context
    // up to max_len (the split count only grows with the context).
    const int step_splits = th::step_attention_splits(s->max_len, s->kv_dtype == TH_KV_BF16,
                                                      (int)(c.num_attention_heads / c.num_key_value_heads),
                                                      (int)c.num_key_value_heads, m->dev->num_cus);
    s->attn_part_floats = th::attention_scratch(1, (size_t)c.num_attention_heads, hd, step_splits);
    for (size_t n = 1; n <= s->fb; ++n) {
        int ns = th::attention_splits(n, (size_t)c.num_attention_heads, (size_t)c.num_key_value_heads, s->max_len, hd);
        s->attn_part_floats =
            std::max(s->attn_part_floats, th::attention_scratch(n, (size_t)c.num_attention_heads, hd, ns));
    }
    if (s->attn_part_floats) TH_HIP(hipMalloc(&s->attn_part, s->attn_part_floats * sizeof(float)));
    if (s->kv_dtype == TH_KV_F32 && s->fb >= th::kGemmMinTokens && hd == 128) {
        s->kv_planes_bytes = th::attention_planes_bytes(s->max_len, (size_t)c.num_key_value_heads);
        TH_HIP(hipMalloc(&s->kv_planes, s->kv_planes_bytes));
        // Zeroed: the attention reads whole 64-key tiles, and the keys of a
        // tile past the context must be finite (they are masked); later
        // writes are splits of finite cached values.
        TH_HIP(hipMemsetAsync(s->kv_planes, 0, s->kv_planes_bytes, m->dev->stream));
    }
    TH_HIP(hipMalloc(&s->argmax_part, th::argmax_partials((size_t)c.vocab_size) * sizeof(uint64_t)));
    TH_HIP(hipMalloc(&s->step, sizeof(th::StepState)));
    s->step_fused = th::step_supported((int)H, (int)I, (int)c.num_attention_heads, (int)c.num_key_value_heads,
                                       (int)hd);
    if (s->step_fused) {
        struct {
            float **p;
            size_t n;
        } sb[] = {{&s->sx_a, H}, {&s->sx_b, H}, {&s->s_y, H}, {&s->s_qkv, qd + 2 * kvd}, {&s->s_att, qd},
                  {&s->s_o, H}, {&s->s_h, I}};
        for (auto &b : sb) TH_HIP(hipMalloc(b.p, b.n * sizeof(float)));
        TH_HIP(hipMalloc(&s->s_part, (size_t)th::step_logits_partials((int)c.vocab_size) * sizeof(uint64_t)));
        // Zeroed: epoch 0 precedes every epoch a step uses. Cleared on the
        // device's stream, which is non-blocking: a null-stream hipMemset
        // would not be ordered before the step kernels.
        const int chunks = std::max(step_reach_chunks(s), 1);
        const size_t words = th::step_qkv_attn_words((int)qd, (int)kvd, (int)c.num_attention_heads, chunks);
        TH_HIP(hipMalloc(&s->s_words, words * sizeof(unsigned long long)));
        TH_HIP(hipMemsetAsync(s->s_words, 0, words * sizeof(unsigned long long), m->dev->stream));
        TH_HIP(hipMalloc(&s->s_err, sizeof(unsigned)));
        TH_HIP(hipMemsetAsync(s->s_err, 0, sizeof(unsigned), m->dev->stream));
    }
    return TH_OK;
}

// What a pick writes for the next step of the fused step kernels: the picked
// token's embedding row, in sx_b.
th::PickEmbed step_embed(th_state *s) {
    th::PickEmbed e;
    if (s->step_fused) {
        e.table = s->m->embed->ptr;
        e.dim = (size_t)s->m->c.hidden_size;
        e.out = s->sx_b;
    }
    return e;
}

// Whether the chunked q/k/v + attention launch takes a step of this state's
// fused decode with `ctx` positions in the context (ctx <= max_len): while
// its chunks (step_reach_chunks) cover the context. That launch is preferred
// while the context's chunks stay at most 16 a head and fewer than 512
// blocks (its blocks past the context leave at once). Past that the streaming launch
// is faster (paired runs, ms a step, chunked -> streaming, the context filling
// the state: Qwen3-0.6B, f32 caches of 1024 positions, 16 chunks: 0.629 ->
// 0.659; 1280: 0.712 -> 0.665; 1536: 0.717 -> 0.683; 2048: 0.784 -> 0.708;
// bf16 caches of 2560: 0.760 -> 0.706; Qwen3-4B, f32 caches of 768
// positions, 384 blocks: 1.904 -> 1.915; 1024, 512 blocks: 1.965 -> 1.939;
// bf16 caches of 2048: 1.967 -> 1.938), while at a short context in a large
// state the chunked launch's blocks past the context leave at once
// (Qwen3-0.6B, 2048 positions, a 16-token context: 0.563 against 0.616 ms).
// So a step takes the chunked launch while its chunks cover the context and
// the streaming launch past that, each in graphs of their own (step_dual).
bool step_chunked(const th_state *s, long long ctx) {
    const long long rows = th::step_qkv_attn_rows(s->kv_dtype == TH_KV_BF16);
    return (std::max(ctx, 1LL) + rows - 1) / rows <= step_reach_chunks(s);
}

// Whether the state keeps two sets of step graphs: the chunked launch's for
// short contexts and the streaming launch's for long ones.
bool step_dual(const th_state *s) {
    return step_chunked(s, 1) && !step_chunked(s, (long long)s->max_len);
}

// Queues one decode step with the fused step kernels: the token and position
// come from s->step, the picked token goes back there. `chunked`: the q/k/v +
// attention take the chunked launch, where the state allows it (step_chunked
// for a short context), or else the streaming one.
int enqueue_step(th_state *s, bool chunked) {
    th_model *m = s->m;
    hipStream_t st = m->dev->stream;
    const th_config &c = m->c;
    const int H = (int)c.hidden_size, I = (int)c.intermediate_size, hd = (int)c.head_dim;
    const int nh = (int)c.num_attention_heads, nkv = (int)c.num_key_value_heads;
    const int qd = nh * hd, kvd = nkv * hd, V = (int)c.vocab_size;
    const float eps = c.rms_norm_eps;
    const int chunks = step_reach_chunks(s);
    const int nsplit = th::step_attention_splits(s->max_len, s->kv_dtype == TH_KV_BF16, nh / nkv, nkv,
                                                 m->dev->num_cus);
    if (th::attention_scratch(1, (size_t)nh, (size_t)hd, nsplit) > s->attn_part_floats)
        return fail(TH_ERR_INVALID, "attention partials exceed the state's scratch");
    // One launch for q/k/v and the chunked attention (step_chunked).
    const bool fuse_attn = chunked && step_chunked(s, 1);
    // Past the chunked launch's reach, the q/k/v GEMV and the streaming
    // attention share a launch when the GEMV blocks are few beside the
    // attention's (Qwen3-0.6B, max_len 4096: 256 GEMV and 1024 attention
    // blocks, 0.876 -> 0.852 ms a step) or when both fit the attention's
    // block slots in one round (Qwen3-0.6B, 4160 positions: 256 + 520 blocks
    // for 1024 slots, 0.829 -> 0.813 ms; a 16-token context in a state of 2200
    // positions: 0.676 -> 0.672 ms). Where they do not (Qwen3-4B at 8192
    // positions: 384 + 688 blocks for 768 slots) the separate launches are
    // faster: 0.2% against the shared launch, and 3% against one whose
    // splits were cut to fit.
    const int gemv_blocks = (qd + 2 * kvd + 15) / 16;
    const bool stream_fused = !fuse_attn && th::step_qkv_attn_supported(H, nh, nkv) && m->layers.size() < 64 &&
                              (3 * gemv_blocks <= nkv * nsplit ||
                               gemv_blocks + nkv * nsplit <= th::step_stream_slots(nh / nkv, s->kv_dtype == TH_KV_BF16,
                                                                                   m->dev->num_cus));
    // sx_b holds the token's embedding row: the previous pick wrote it.
    const float *y_prev = nullptr;
    for (size_t l = 0; l < m->layers.size(); ++l) {
        const Layer &L = m->layers[l];
        th::StepQkvArgs q{};
        q.wq = L.q->ptr;
        q.wk = L.k->ptr;
        q.wv = L.v->ptr;
        q.q_rows = qd;
        q.kv_rows = kvd;
        q.hidden = H;
        q.x_prev = s->sx_b;
        q.y_prev = y_prev;
        q.gain = L.attn_norm->ptr;
        q.eps = eps;
        q.x_out = s->sx_a;
        q.qkv = s->s_qkv;
        th::StepAttnArgs a{};
        a.qkv = s->s_qkv;
        a.q_norm = L.q_norm ? L.q_norm->ptr : nullptr;
        a.k_norm = L.k_norm ? L.k_norm->ptr : nullptr;
        a.rope = s->rope->ptr;
        a.k_cache = cache_ptr(s, l, 0);
        a.v_cache = cache_ptr(s, l, 1);
        a.head_stride = (long long)(s->max_len * hd);
        a.pos = &s->step->pos;
        a.n_heads = nh;
        a.n_kv_heads = nkv;
        a.nsplit = fuse_attn ? 1 : nsplit;
        a.kv_bf16 = s->kv_dtype == TH_KV_BF16;
        a.eps = eps;
        a.out = s->s_att;
        a.part_acc = s->attn_part;
        a.part_ml = s->attn_part ? s->attn_part + (size_t)nh * nsplit * hd : nullptr;
        if (fuse_attn) {
            th::StepQkvAttnArgs f{};
            f.qkv = q;
            f.at = a;
            f.words = s->s_words;
            f.err = s->s_err;
            f.st = s->step;
            f.layer = (int)l;
            f.chunks = chunks;
            TH_HIP(th::launch_step_qkv_attn(st, f));
        } else if (stream_fused) {
            // Past the chunked launch's reach: the q/k/v GEMV and the
            // streaming split attention in one launch, then the combine.
            th::StepQkvAttnArgs f{};
            f.qkv = q;
            f.at = a;
            f.words = s->s_words;
            f.err = s->s_err;
            f.st = s->step;
            f.layer = (int)l;
            TH_HIP(th::launch_step_qkv_stream(st, f));
            if (nsplit > 1)
                TH_HIP(th::launch_attn_combine(st, s->s_att, a.part_acc, a.part_ml, (size_t)nh, nsplit, hd));
        } else {
            TH_HIP(th::launch_step_qkv(st, q));
            TH_HIP(th::launch_step_attention(st, a));
            if (nsplit > 1)
                TH_HIP(th::launch_attn_combine(st, s->s_att, a.part_acc, a.part_ml, (size_t)nh, nsplit, hd));
        }
        TH_HIP(th::launch_step_gemv(st, L.o->ptr, H, qd, s->s_att, s->s_o));
        TH_HIP(th::launch_step_gate_up(st, L.gate->ptr, L.up->ptr, I, H, s->sx_a, s->s_o, L.mlp_norm->ptr, eps,
                                       s->sx_b, s->s_h));
        TH_HIP(th::launch_step_gemv(st, L.down->ptr, H, I, s->s_h, s->s_y));
        y_prev = s->s_y;
    }
    int np = 0;
    TH_HIP(th::launch_step_logits(st, m->out_proj()->ptr, V, H, s->sx_b, y_prev, m->norm->ptr, eps,
                                  s->logits->ptr, s->s_part, &np));
    if (s->graph_keep) TH_HIP(th::launch_keep_logits(st, s->logits->ptr, (size_t)V, s->step));
    if (s->sampling)
        TH_HIP(th::launch_sample(st, s->logits->ptr, (size_t)V, s->s_cand, s->s_sample, s->step, 1, step_embed(s)));
    else
        TH_HIP(th::launch_pick_partials(st, s->s_part, (size_t)np, s->step, 1, step_embed(s)));
    return TH_OK;
}

// Queues the fused forward of n tokens (n <= s->fb) at position pos, or at
// *pos_dev when pos_dev is not null (a captured decode step). Token ids are
// read from the device array `tokens`. Leaves the logits of the last token in
// s->logits.
int enqueue_fused(th_state *s, const uint32_t *tokens, size_t n, size_t pos, const long long *pos_dev) {
    th_model *m = s->m;
    th_device *d = m->dev;
    hipStream_t st = d->stream;
    const th_config &c = m->c;
    const float eps = c.rms_norm_eps;
    const size_t H = (size_t)c.hidden_size, I = (size_t)c.intermediate_size, hd = (size_t)c.head_dim;
    const size_t nh = (size_t)c.num_attention_heads, nkv = (size_t)c.num_key_value_heads;
    const size_t qd = nh * hd;
    const int kv_bf16 = s->kv_dtype == TH_KV_BF16;
    const size_t max_ctx = pos_dev ? s->max_len : pos + n;
    const int nsplit = th::attention_splits(n, nh, nkv, max_ctx, hd);
    if (th::attention_scratch(n, nh, hd, nsplit) > s->attn_part_floats)
        return fail(TH_ERR_INVALID, "attention partials exceed the state's scratch");
    // Chunks of kGemmMinTokens or more go through the MFMA GEMM (activations
    // split once per input into fsplit).
    auto use_gemm = [&](size_t cols) { return n >= th::kGemmMinTokens && s->fsplit && cols <= s->fsplit_cols; };

    // When every projection goes through the MFMA GEMM, the kernels that
    // produce a GEMM input (the norms, attention, silu_mul) write it as bf16
    // hi/lo terms directly, and the residual add after the o and down GEMMs
    // sums their split-K partials itself.
    const bool hl = use_gemm(std::max(std::max(H, qd), I)) && th::gemm_supported(qd, H) &&
                    th::gemm_supported(nkv * hd, H) && th::gemm_supported(H, qd) && th::gemm_supported(I, H) &&
                    th::gemm_supported(H, I);
    uint16_t *hi = static_cast<uint16_t *>(s->fsplit), *lo = hi ? hi + s->fb * s->fsplit_cols : nullptr;
    float *part = hi ? reinterpret_cast<float *>(hi + 2 * s->fb * s->fsplit_cols) : nullptr;
    const int ks_o = th::gemm_ksplit(n, H, qd, 1), ks_down = th::gemm_ksplit(n, H, I, 1);
    // The residual still to be added to fx: ny partials of stride y_stride.
    const float *res = nullptr;
    int nres = 0;
    size_t res_stride = 0;
    auto single_gemm = [&](const uint16_t *w, size_t cols, int ks, const uint16_t *xh, const uint16_t *xl) -> int {
        const th::GemmOut o{w, H, s->fy};
        TH_HIP(th::launch_gemm_hl(st, xh, xl, n, cols, &o, 1, part, ks));
        res = ks > 1 ? part : s->fy;
        nres = ks;
        res_stride = n * H;
        return TH_OK;
    };

    TH_HIP(th::launch_embed(st, s->fx, m->embed->ptr, H, tokens, n));
    for (size_t i = 0; i < m->layers.size(); ++i) {
        const Layer &L = m->layers[i];
        th::QkvPostArgs qa{};
        qa.q = s->fq;
        qa.k = s->fk;
        qa.v = s->fv;
        qa.q_norm = L.q_norm ? L.q_norm->ptr : nullptr;
        qa.k_norm = L.k_norm ? L.k_norm->ptr : nullptr;
        qa.rope = s->rope->ptr;
        qa.k_cache = cache_ptr(s, i, 0);
        qa.v_cache = cache_ptr(s, i, 1);
        qa.head_stride = (long long)(s->max_len * hd);
        qa.pos_stride = (long long)hd;
        qa.pos = (long long)pos;
        qa.pos_dev = pos_dev;
        qa.n = (int)n;
        qa.n_heads = (int)nh;
        qa.n_kv_heads = (int)nkv;
        qa.head_dim = (int)hd;
        qa.kv_bf16 = kv_bf16;
        qa.eps = eps;
        th::AttnKernelArgs aa{};
        aa.out = s->fatt;
        aa.q = s->fq;
        aa.k = qa.k_cache;
        aa.v = qa.v_cache;
        aa.n_heads = (int)nh;
        aa.n_kv_heads = (int)nkv;
        aa.group = (int)(nh / nkv);
        aa.pos = (long long)pos;
        aa.pos_dev = pos_dev;
        aa.pos_stride = (long long)hd;
        aa.head_stride = (long long)(s->max_len * hd);
        aa.nsplit = nsplit;
        aa.kv_bf16 = kv_bf16;
        aa.scale = 1.0f / sqrtf((float)hd);
        aa.part_acc = s->attn_part;
        aa.part_ml = s->attn_part ? s->attn_part + n * nh * (size_t)nsplit * hd : nullptr;
        if (hl) {
            aa.out_hi = hi;
            aa.out_lo = lo;
        }
        // The attention through bf16 planes of the keys and values (f32
        // caches); the fused q/k/v GEMM writes the new positions' planes in
        // its epilogue.
        const bool use_planes = s->kv_planes && th::attention_planes_supported(aa, n, hd);
        bool planes_written = false;
        // Residual add of the previous layer's MLP output, then the attention norm.
        if (hl) {
            TH_HIP(th::launch_add_rmsnorm_parts(st, s->fx, res, nres, res_stride, nullptr, hi, lo, n,
                                                L.attn_norm->ptr, H, eps));
            // The q/k/v GEMMs with the q/k norm + RoPE + KV append epilogue,
            // which also writes the new positions' planes.
            auto epilogue_planes = [&]() -> int {
                if (!use_planes) return TH_OK;
                // Earlier positions from the caches first (its zeros past
                // them precede the epilogue's writes).
                TH_HIP(th::launch_kv_planes(st, aa, pos, s->kv_planes, s->kv_planes_bytes, s->max_len));
                const th::PlanePtrs pp = th::attention_planes_of(s->kv_planes, s->max_len, nkv);
                qa.kh = pp.kh;
                qa.kl = pp.kl;
                qa.vh = pp.vh;
                qa.vl = pp.vl;
                qa.plane_len = pp.plane_len;
                planes_written = true;
                return TH_OK;
            };
            if (th::gemm_qkv_fused(n, qd, nkv * hd, H, hd)) {
                TRY(epilogue_planes());
                TH_HIP(th::launch_gemm_qkv(st, hi, lo, H, L.q->ptr, L.k->ptr, L.v->ptr, qa));
            } else if (!pos_dev && th::gemm_qkv_huge_fused(n, qd, nkv * hd, H, hd, (long long)pos)) {
                TRY(epilogue_planes());
                TH_HIP(th::launch_gemm_qkv_huge(st, hi, lo, H, L.q->ptr, L.k->ptr, L.v->ptr, qa));
            } else {
                const th::GemmOut o[3] = {
                    {L.q->ptr, qd, s->fq}, {L.k->ptr, nkv * hd, s->fk}, {L.v->ptr, nkv * hd, s->fv}};
                TH_HIP(th::launch_gemm_hl(st, hi, lo, n, H, o, 3, nullptr, 1));
                TH_HIP(th::launch_qk_norm_rope_append(st, qa));
            }
        } else {
            TH_HIP(th::launch_add_rmsnorm(st, s->fx, i ? s->fy : nullptr, s->fxb, n, L.attn_norm->ptr, H, eps));
            if (use_gemm(H) && th::gemm_supported(qd, H) && th::gemm_supported(nkv * hd, H)) {
                const th::GemmOut o[3] = {
                    {L.q->ptr, qd, s->fq}, {L.k->ptr, nkv * hd, s->fk}, {L.v->ptr, nkv * hd, s->fv}};
                TH_HIP(th::launch_gemm_multi(st, s->fxb, n, H, o, 3, s->fsplit, s->fsplit_bytes));
            } else {
                TH_HIP(th::launch_matmul(st, s->fq, L.q->ptr, qd, H, s->fxb, n));
                TH_HIP(th::launch_matmul(st, s->fk, L.k->ptr, nkv * hd, H, s->fxb, n));
                TH_HIP(th::launch_matmul(st, s->fv, L.v->ptr, nkv * hd, H, s->fxb, n));
            }
            TH_HIP(th::launch_qk_norm_rope_append(st, qa));
        }

        if (use_planes)
            TH_HIP(th::launch_attention_planes(st, aa, n, hd, s->kv_planes, s->kv_planes_bytes, s->max_len,
                                               !planes_written));
        else
            TH_HIP(th::launch_attention(st, aa, n, hd));

        if (hl) {
            TRY(single_gemm(L.o->ptr, qd, ks_o, hi, lo));
            TH_HIP(th::launch_add_rmsnorm_parts(st, s->fx, res, nres, res_stride, nullptr, hi, lo, n,
                                                L.mlp_norm->ptr, H, eps));
            if (I % 64 == 0) {
                // gate/up with the SiLU * up epilogue, whose hi/lo output takes
                // fgate's bytes (fb x I x 4).
                uint16_t *h_hi = reinterpret_cast<uint16_t *>(s->fgate), *h_lo = h_hi + s->fb * I;
                TH_HIP(th::launch_gemm_silu(st, hi, lo, n, H, L.gate->ptr, L.up->ptr, I, h_hi, h_lo));
                TRY(single_gemm(L.down->ptr, I, ks_down, h_hi, h_lo));
            } else {
                const th::GemmOut o[2] = {{L.gate->ptr, I, s->fgate}, {L.up->ptr, I, s->fup}};
                TH_HIP(th::launch_gemm_hl(st, hi, lo, n, H, o, 2, nullptr, 1));
                TH_HIP(th::launch_silu_mul_split(st, s->fgate, s->fup, n * I, hi, lo));
                TRY(single_gemm(L.down->ptr, I, ks_down, hi, lo));
            }
            continue;
        }
        if (use_gemm(qd) && th::gemm_supported(H, qd)) {
            const th::GemmOut o{L.o->ptr, H, s->fy};
            TH_HIP(th::launch_gemm_multi(st, s->fatt, n, qd, &o, 1, s->fsplit, s->fsplit_bytes));
        } else {
            TH_HIP(th::launch_matmul(st, s->fy, L.o->ptr, H, qd, s->fatt, n));
        }
        TH_HIP(th::launch_add_rmsnorm(st, s->fx, s->fy, s->fxb, n, L.mlp_norm->ptr, H, eps));
        if (use_gemm(H) && th::gemm_supported(I, H)) {
            const th::GemmOut o[2] = {{L.gate->ptr, I, s->fgate}, {L.up->ptr, I, s->fup}};
            TH_HIP(th::launch_gemm_multi(st, s->fxb, n, H, o, 2, s->fsplit, s->fsplit_bytes));
        } else {
            TH_HIP(th::launch_matmul(st, s->fgate, L.gate->ptr, I, H, s->fxb, n));
            TH_HIP(th::launch_matmul(st, s->fup, L.up->ptr, I, H, s->fxb, n));
        }
        TH_HIP(th::launch_silu_mul(st, s->fgate, s->fup, n * I));
        if (use_gemm(I) && th::gemm_supported(H, I)) {
            const th::GemmOut o{L.down->ptr, H, s->fy};
            TH_HIP(th::launch_gemm_multi(st, s->fgate, n, I, &o, 1, s->fsplit, s->fsplit_bytes));
        } else {
            TH_HIP(th::launch_matmul(st, s->fy, L.down->ptr, H, I, s->fgate, n));
        }
        res = s->fy;
        nres = 1;
        res_stride = 0;
    }
    // Only the last token's logits are wanted (model.rs:143-147).
    float *xl = s->fx + (n - 1) * H;
    TH_HIP(th::launch_add_rmsnorm_parts(st, xl, res ? res + (n - 1) * H : nullptr, nres, res_stride, s->fxb, nullptr,
                                        nullptr, 1, m->norm->ptr, H, eps));
    TH_HIP(th::launch_matmul(st, s->logits->ptr, m->out_proj()->ptr, (size_t)c.vocab_size, H, s->fxb, 1));
    return TH_OK;
}

int stage_state_tokens(th_state *s, const uint32_t *tokens, size_t n) {
    th_model *m = s->m;
    for (size_t i = 0; i < n; ++i)
        if (tokens[i] >= (uint32_t)m->c.vocab_size)
            return fail(TH_ERR_INVALID, "token %u at index %zu is past the vocabulary of %lld", tokens[i], i,
                        (long long)m->c.vocab_size);
    if (n > s->tokens_dev_cap) {
        TH_HIP(hipStreamSynchronize(m->dev->stream));
        free_dev(s->tokens_dev);
        s->tokens_dev = nullptr;
        s->tokens_dev_cap = 0;
        size_t cap = std::max<size_t>(n, 1024);
        TH_HIP(hipMalloc(&s->tokens_dev, cap * sizeof(uint32_t)));
        s->tokens_dev_cap = cap;
    }
    TH_HIP(hipMemcpyAsync(s->tokens_dev, tokens, n * sizeof(uint32_t), hipMemcpyHostToDevice, m->dev->stream));
    return TH_OK;
}

// The ops and trait paths share the reference's caches; the fused path keeps
// its own.
int claim_path(th_state *s, int path) {
    const int layout = path == TH_PATH_TRAIT ? TH_PATH_OPS : path;
    if (s->path != -1 && s->path != layout)
        return fail(TH_ERR_INVALID, "this state's caches were filled by the other path");
    if (layout == TH_PATH_OPS && s->kv_dtype != TH_KV_F32)
        return fail(TH_ERR_INVALID, "the ops and trait paths keep the reference's f32 caches");
    s->path = layout;
    return TH_OK;
}

// Decode steps per replay of the multi-step graph: a replay boundary costs
// the GPU ≈6 µs against ≈1.5 µs between kernels inside a graph (0.6B decode:
// 0.619 -> 0.6145 ms a step with 4 steps a replay). Longer replays measured
// slower: 0.562-0.563 ms a step with 8, 0.566-0.567 with 16, 0.571 with 32.
constexpr size_t kGraphSteps = 8;

// Captures `n_steps` decode steps (n = 1 each, position and token from
// s->step) as one graph; `chunked` as enqueue_step takes it.
int capture_steps(th_state *s, size_t n_steps, bool chunked, hipGraph_t *graph, hipGraphExec_t *exec) {
    if (*exec) return TH_OK;
    th_model *m = s->m;
    hipStream_t st = m->dev->stream;
    const size_t vocab = (size_t)m->c.vocab_size;
    TH_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    int rc = TH_OK;
    for (size_t k = 0; k < n_steps && rc == TH_OK; ++k) {
        if (s->step_fused) {
            rc = enqueue_step(s, chunked);
        } else {
            const long long *pos_dev = &s->step->pos;
            const uint32_t *tok_dev = &s->step->token;
            rc = enqueue_fused(s, tok_dev, 1, 0, pos_dev);
            if (rc == TH_OK) {
                hipError_t e = s->graph_keep ? th::launch_keep_logits(st, s->logits->ptr, vocab, s->step) : hipSuccess;
                if (e == hipSuccess)
                    e = s->sampling ? th::launch_sample(st, s->logits->ptr, vocab, s->s_cand, s->s_sample, s->step, 1)
                                    : th::launch_pick(st, s->logits->ptr, vocab, s->argmax_part, s->step, 1);
                if (e != hipSuccess) rc = fail(TH_ERR_HIP, "capture: %s", hipGetErrorString(e));
            }
        }
    }
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(st, &g);
    if (rc != TH_OK) {
        if (g) (void)hipGraphDestroy(g);
        return rc;
    }
    if (e != hipSuccess) return fail(TH_ERR_HIP, "hipStreamEndCapture: %s", hipGetErrorString(e));
    *graph = g;
    TH_HIP(hipGraphInstantiate(exec, g, nullptr, nullptr, 0));
    return TH_OK;
}

// Whether the decode steps fed at positions [pos, pos + n) take the chunked
// launch's graphs of a state that keeps both (the context at the last of them
// is at most pos + n: a step advances the position by one at most).
bool steps_chunked(const th_state *s, size_t pos, size_t n) { return step_chunked(s, (long long)(pos + n)); }

// Queues `n` decode steps fed from position `pos` on (the graphs captured by
// capture_or_keep): replays of the multi-step graph, then of the one-step
// graph for the rest, each from the chunked or the streaming set by the
// context it can reach.
int launch_steps(th_state *s, size_t pos, size_t n) {
    hipStream_t st = s->m->dev->stream;
    TH_REQUIRE(s->graph_exec && s->graph_n_exec, "decode steps launched before their capture");
    const bool dual = s->graph_l_exec != nullptr;
    for (; n >= kGraphSteps; n -= kGraphSteps, pos += kGraphSteps)
        TH_HIP(hipGraphLaunch(dual && !steps_chunked(s, pos, kGraphSteps) ? s->graph_ln_exec : s->graph_n_exec, st));
    for (; n; --n, ++pos)
        TH_HIP(hipGraphLaunch(dual && !steps_chunked(s, pos, 1) ? s->graph_l_exec : s->graph_exec, st));
    return TH_OK;
}

// The captured decode steps (one, and kGraphSteps), captured again unless
// they already copy out the logits as `keep` asks and draw or pick as
// `sampling` asks. Captured before the call queues any step work.
int capture_or_keep(th_state *s, bool keep, bool sampling) {
    if (s->graph_keep != keep || s->sampling != sampling) {
        if (s->graph_exec) TH_HIP(hipGraphExecDestroy(s->graph_exec));
        if (s->graph) TH_HIP(hipGraphDestroy(s->graph));
        if (s->graph_n_exec) TH_HIP(hipGraphExecDestroy(s->graph_n_exec));
        if (s->graph_n) TH_HIP(hipGraphDestroy(s->graph_n));
        if (s->graph_l_exec) TH_HIP(hipGraphExecDestroy(s->graph_l_exec));
        if (s->graph_l) TH_HIP(hipGraphDestroy(s->graph_l));
        if (s->graph_ln_exec) TH_HIP(hipGraphExecDestroy(s->graph_ln_exec));
        if (s->graph_ln) TH_HIP(hipGraphDestroy(s->graph_ln));
        s->graph_exec = nullptr;
        s->graph = nullptr;
        s->graph_n_exec = nullptr;
        s->graph_n = nullptr;
        s->graph_l_exec = nullptr;
        s->graph_l = nullptr;
        s->graph_ln_exec = nullptr;
        s->graph_ln = nullptr;
    }
    s->graph_keep = keep;
    s->sampling = sampling;
    // The default set: the chunked launch where the state allows it for a
    // short context; a state that keeps both also gets the streaming set.
    const bool chunked = step_chunked(s, 1);
    TRY(capture_steps(s, 1, chunked, &s->graph, &s->graph_exec));
    TRY(capture_steps(s, kGraphSteps, chunked, &s->graph_n, &s->graph_n_exec));
    if (!s->step_fused || !step_dual(s)) return TH_OK;
    TRY(capture_steps(s, 1, false, &s->graph_l, &s->graph_l_exec));
    return capture_steps(s, kGraphSteps, false, &s->graph_ln, &s->graph_ln_exec);
}

}  // namespace

extern "C" {

int th_model_create(th_device *dev, const th_config *config, const th_weight *const *weights, size_t n_weights,
                    th_model **out) {
    TH_REQUIRE(dev && config && weights && out, "th_model_create: null argument");
    TH_NOT_CAPTURING(dev, "th_model_create");
    const th_config &c = *config;
    TH_REQUIRE(c.hidden_size > 0 && c.intermediate_size > 0 && c.num_hidden_layers > 0 && c.num_attention_heads > 0 &&
                   c.num_key_value_heads > 0 && c.head_dim > 0 && c.vocab_size > 0,
               "config sizes must be positive");
    TH_REQUIRE(c.num_attention_heads % c.num_key_value_heads == 0, "query heads must split into KV groups");
    TH_REQUIRE(c.num_attention_heads / c.num_key_value_heads <= 8, "at most 8 query heads per KV head");
    TH_REQUIRE(c.head_dim == 64 || c.head_dim == 128 || c.head_dim == 256, "head_dim must be 64, 128 or 256");
    TH_REQUIRE(c.hidden_size % 8 == 0 && c.intermediate_size % 8 == 0, "hidden and MLP sizes must be multiples of 8");
    size_t L = (size_t)c.num_hidden_layers;
    TH_REQUIRE(n_weights == L * kWeightsPerLayer + 3, "expected %zu weights, got %zu", L * kWeightsPerLayer + 3,
               n_weights);
    const size_t H = (size_t)c.hidden_size, I = (size_t)c.intermediate_size, hd = (size_t)c.head_dim;
    const size_t qd = (size_t)c.num_attention_heads * hd, kvd = (size_t)c.num_key_value_heads * hd;
    auto *m = new (std::nothrow) th_model();
    if (!m) return fail(TH_ERR_NOMEM, "out of host memory");
    m->dev = dev;
    m->c = c;
    int rc = TH_OK;
    for (size_t l = 0; l < L && rc == TH_OK; ++l) {
        const th_weight *const *w = weights + l * kWeightsPerLayer;
        Layer lay{w[0], w[1], w[2], w[3], w[4], w[5], w[6], w[7], w[8], w[9], w[10]};
        if (!rc) rc = check_shape(lay.attn_norm, H, 0, "input_layernorm", l);
        if (!rc) rc = check_shape(lay.q, qd, H, "q_proj", l);
        if (!rc) rc = check_shape(lay.k, kvd, H, "k_proj", l);
        if (!rc) rc = check_shape(lay.v, kvd, H, "v_proj", l);
        if (!rc) rc = check_shape(lay.o, H, qd, "o_proj", l);
        if (!rc && lay.q_norm) rc = check_shape(lay.q_norm, hd, 0, "q_norm", l);
        if (!rc && lay.k_norm) rc = check_shape(lay.k_norm, hd, 0, "k_norm", l);
        if (!rc) rc = check_shape(lay.mlp_norm, H, 0, "post_attention_layernorm", l);
        if (!rc) rc = check_shape(lay.gate, I, H, "gate_proj", l);
        if (!rc) rc = check_shape(lay.up, I, H, "up_proj", l);
        if (!rc) rc = check_shape(lay.down, H, I, "down_proj", l);
        m->layers.push_back(lay);
    }
    const th_weight *const *tail = weights + L * kWeightsPerLayer;
    m->embed = tail[0];
    m->norm = tail[1];
    m->lm_head = tail[2];
    if (!rc) rc = check_shape(m->embed, (size_t)c.vocab_size, H, "embed_tokens", L);
    if (!rc) rc = check_shape(m->norm, H, 0, "norm", L);
    if (!rc && c.tie_word_embeddings && m->lm_head) rc = fail(TH_ERR_INVALID, "tied embeddings take no lm_head");
    if (!rc && !c.tie_word_embeddings) rc = check_shape(m->lm_head, (size_t)c.vocab_size, H, "lm_head", L);
    if (rc) {
        delete m;
        return rc;
    }
    *out = m;
    return TH_OK;
}

void th_model_destroy(th_model *m) {
    if (!m) return;
    if (m->dev->capturing) {  // the handle stays valid: destroy it after th_graph_end
        th::fail(TH_ERR_INVALID, "th_model_destroy cannot run while the device's stream is being captured");
        return;
    }
    for (th_weight *w : m->owned) th_weight_free(m->dev, w);
    delete m;
}

int th_model_config(const th_model *m, th_config *out) {
    TH_REQUIRE(m && out, "th_model_config: null argument");
    *out = m->c;
    return TH_OK;
}

int th_state_create(th_model *m, size_t max_len, int kv_dtype, th_state **out) {
    TH_REQUIRE(m && out, "th_state_create: null argument");
    TH_NOT_CAPTURING(m->dev, "th_state_create");
    TH_REQUIRE(max_len > 0, "max_len must be positive");
    TH_REQUIRE(kv_dtype == TH_KV_F32 || kv_dtype == TH_KV_BF16, "unknown KV dtype %d", kv_dtype);
    auto *s = new (std::nothrow) th_state();
    if (!s) return fail(TH_ERR_NOMEM, "out of host memory");
    s->m = m;
    s->max_len = max_len;
    s->kv_dtype = kv_dtype;
    std::vector<float> table = rope_table(max_len, (size_t)m->c.head_dim, m->c.rope_theta);
    int rc = th_alloc(m->dev, table.size(), &s->rope);
    if (!rc) rc = th_write(m->dev, s->rope, table.data(), table.size());
    if (!rc) rc = th_alloc(m->dev, (size_t)m->c.vocab_size, &s->logits);
    if (rc) {
        th_state_destroy(s);
        return rc;
    }
    *out = s;
    return TH_OK;
}

void th_state_destroy(th_state *s) {
    if (!s) return;
    th_device *d = s->m->dev;
    if (d->capturing) {  // the handle stays valid: destroy it after th_graph_end
        th::fail(TH_ERR_INVALID, "th_state_destroy cannot run while the device's stream is being captured");
        return;
    }
    (void)hipStreamSynchronize(d->stream);
    if (s->graph_exec) (void)hipGraphExecDestroy(s->graph_exec);
    if (s->graph) (void)hipGraphDestroy(s->graph);
    if (s->graph_n_exec) (void)hipGraphExecDestroy(s->graph_n_exec);
    if (s->graph_n) (void)hipGraphDestroy(s->graph_n);
    if (s->graph_l_exec) (void)hipGraphExecDestroy(s->graph_l_exec);
    if (s->graph_l) (void)hipGraphDestroy(s->graph_l);
    if (s->graph_ln_exec) (void)hipGraphExecDestroy(s->graph_ln_exec);
    if (s->graph_ln) (void)hipGraphDestroy(s->graph_ln);
    th_buffer *bufs[] = {s->rope, s->logits, s->x, s->xb, s->q, s->k, s->v, s->att, s->gate, s->up};
    for (th_buffer *b : bufs) th_buffer_free(d, b);
    for (th_buffer *b : s->k_cache) th_buffer_free(d, b);
    for (th_buffer *b : s->v_cache) th_buffer_free(d, b);
    void *ptrs[] = {s->fx,      s->fxb,        s->fq,   s->fk,         s->fv,         s->fatt,
                    s->fgate,   s->fup,        s->fy,   s->kv,         s->attn_part,  s->argmax_part,
                    s->step,    s->tokens_dev, s->logits_dev, s->sx_a, s->sx_b, s->s_y, s->s_qkv,
                    s->s_att, s->s_o, s->s_h, s->s_part, s->s_words, s->s_err, s->fsplit, s->s_sample,
                    s->s_cand, s->kv_planes};
    for (void *p : ptrs) free_dev(p);
    delete s;
}

int th_forward(th_model *m, th_state *s, const uint32_t *tokens, size_t n, size_t pos, float *logits, int path) {
    TH_REQUIRE(m && s && s->m == m, "th_forward: null argument or a state of another model");
    TH_NOT_CAPTURING(m->dev, "th_forward");
    TH_REQUIRE(n > 0 && tokens, "no tokens to run");  // model.rs:84
    TH_REQUIRE(pos + n <= s->max_len, "tokens past the end of the cache");  // model.rs:85
    TH_REQUIRE(path == TH_PATH_OPS || path == TH_PATH_FUSED || path == TH_PATH_TRAIT, "unknown path %d", path);
    TRY(claim_path(s, path));
    if (path == TH_PATH_OPS) {
        TRY(ensure_ops_state(s));
        for (size_t i = 0; i < n; i += kBatch) TRY(forward_batch_ops(s, tokens + i, std::min(kBatch, n - i), pos + i));
    } else if (path == TH_PATH_TRAIT) {
        TRY(ensure_ops_state(s));
        for (size_t i = 0; i < n; i += kBatch)
            TRY(forward_batch_trait(s, tokens + i, std::min(kBatch, n - i), pos + i));
    } else {
        TRY(ensure_fused_state(s));
        TRY(stage_state_tokens(s, tokens, n));
        for (size_t i = 0; i < n; i += s->fb)
            TRY(enqueue_fused(s, s->tokens_dev + i, std::min(s->fb, n - i), pos + i, nullptr));
    }
    if (logits) return th_read(m->dev, s->logits, logits, s->logits->len);
    TH_HIP(hipStreamSynchronize(m->dev->stream));
    return TH_OK;
}

}  // extern "C"

namespace {

// Decode steps a call with stop tokens enqueues between looks at whether one
// has been picked (the steps after it repeat the last one and are wasted).
constexpr size_t kStopCheckSteps = 8;

// th_decode, and th_decode_sample when `sp` (the sampler's parameters and
// generator state, updated on return) is not null. With stop tokens the call
// ends at the first pick among them (recorded, not fed); *n_out then counts
// the tokens written to out_tokens, the stop token included.
int decode(th_model *m, th_state *s, size_t pos, size_t steps, uint32_t *out_tokens, float *out_logits,
           th::SampleState *sp, const uint32_t *stops = nullptr, size_t n_stop = 0, size_t *n_out = nullptr,
           bool *hit_stop = nullptr) {
    if (hit_stop) *hit_stop = false;
    TH_REQUIRE(m && s && s->m == m && out_tokens, "th_decode: null argument or a state of another model");
    TH_NOT_CAPTURING(m->dev, "th_decode");
    TH_REQUIRE(n_stop <= (size_t)th::kStepMaxStops && (n_stop == 0 || stops), "at most %d stop tokens",
               th::kStepMaxStops);
    if (n_out) *n_out = 0;
    TH_REQUIRE(s->path == TH_PATH_FUSED, "decode continues a fused-path forward; run th_forward first");
    TH_REQUIRE(pos + steps <= s->max_len, "tokens past the end of the cache");
    if (steps == 0) return TH_OK;
    th_device *d = m->dev;
    hipStream_t st = d->stream;
    const size_t vocab = (size_t)m->c.vocab_size;
    TRY(ensure_fused_state(s));
    const bool sampling = sp != nullptr;
    if (sampling && !s->s_sample) {
        TH_HIP(hipStreamSynchronize(st));
        TH_HIP(hipMalloc(&s->s_sample, sizeof(th::SampleState)));
        TH_HIP(hipMalloc(&s->s_cand, th::sample_scratch_bytes(vocab)));
    }
    if (steps + 1 > s->tokens_dev_cap) {
        TH_HIP(hipStreamSynchronize(st));
        free_dev(s->tokens_dev);
        s->tokens_dev = nullptr;
        s->tokens_dev_cap = 0;
        TH_HIP(hipMalloc(&s->tokens_dev, (steps + 1) * sizeof(uint32_t)));
        s->tokens_dev_cap = steps + 1;
    }
    if (out_logits && steps * vocab > s->logits_dev_cap) {
        TH_HIP(hipStreamSynchronize(st));
        free_dev(s->logits_dev);
        s->logits_dev = nullptr;
        s->logits_dev_cap = 0;
        TH_HIP(hipMalloc(&s->logits_dev, steps * vocab * sizeof(float)));
        s->logits_dev_cap = steps * vocab;
    }
    th::StepState init{};
    init.pos = (long long)pos;
    init.step = 0;
    init.tokens_out = s->tokens_dev;
    init.logits_out = out_logits ? s->logits_dev : nullptr;
    init.epoch = s->step_epoch;
    init.n_stop = (int)n_stop;
    for (size_t i = 0; i < n_stop; ++i) init.stop[i] = stops[i];
    TH_HIP(hipMemcpyAsync(s->step, &init, sizeof init, hipMemcpyHostToDevice, st));
    if (sampling) TH_HIP(hipMemcpyAsync(s->s_sample, sp, sizeof *sp, hipMemcpyHostToDevice, st));
    TH_HIP(hipStreamSynchronize(st));  // `init` is a stack temporary
    const char *mode = getenv("TITANIA_DECODE");
    // The first pick comes from the logits the last forward left.
    auto first_pick = [&]() {
        return sampling ? th::launch_sample(st, s->logits->ptr, vocab, s->s_cand, s->s_sample, s->step, 0,
                                            step_embed(s))
                        : th::launch_pick(st, s->logits->ptr, vocab, s->argmax_part, s->step, 0, step_embed(s));
    };
    // Whether a stop token has been picked (its index in tokens_out + 1).
    int stopped = 0;
    auto look = [&]() -> int {
        TH_HIP(hipMemcpyAsync(&stopped, &s->step->stopped, sizeof stopped, hipMemcpyDeviceToHost, st));
        TH_HIP(hipStreamSynchronize(st));
        return TH_OK;
    };
    size_t launched = 0;  // steps enqueued (each advances the epoch once)
    if (n_stop) {
        // The loop of model/chat.rs:147-178 on the device: the captured step,
        // a few steps at a time, until a stop token or `steps` tokens.
        TRY(capture_or_keep(s, out_logits != nullptr, sampling));
        TH_HIP(first_pick());
        TRY(look());
        while (!stopped && launched < steps) {
            const size_t n = std::min(kStopCheckSteps, steps - launched);
            TRY(launch_steps(s, pos + launched, n));
            launched += n;
            TRY(look());
        }
    } else if (mode && strcmp(mode, "eager") == 0 && s->step_fused) {
        // The same step kernels launched one by one (no graph): for profilers
        // that do not follow graph launches.
        s->graph_keep = out_logits != nullptr;
        s->sampling = sampling;
        TH_HIP(first_pick());
        for (size_t i = 0; i < steps; ++i) TRY(enqueue_step(s, step_chunked(s, (long long)(pos + i + 1))));
        launched = steps;
    } else {
        TRY(capture_or_keep(s, out_logits != nullptr, sampling));
        TH_HIP(first_pick());
        TRY(launch_steps(s, pos, steps));
        launched = steps;
    }
    s->step_epoch += (uint32_t)launched;
    // A stop token picked after the last fed token is past the call's tokens:
    // the next call picks it again.
    if ((size_t)stopped > steps) stopped = 0;
    if (hit_stop) *hit_stop = stopped != 0;
    // Tokens out: all `steps`, or up to the stop token; each but the stop
    // token was fed, and its logits kept when asked.
    const size_t n_tok = stopped ? (size_t)stopped : steps;
    const size_t n_fed = stopped ? (size_t)stopped - 1 : steps;
    if (n_out) *n_out = n_tok;
    TH_HIP(hipMemcpyAsync(out_tokens, s->tokens_dev, n_tok * sizeof(uint32_t), hipMemcpyDeviceToHost, st));
    if (out_logits && n_fed)
        TH_HIP(hipMemcpyAsync(out_logits, s->logits_dev, n_fed * vocab * sizeof(float), hipMemcpyDeviceToHost, st));
    unsigned poll_failures = 0;
    if (s->s_err) TH_HIP(hipMemcpyAsync(&poll_failures, s->s_err, sizeof poll_failures, hipMemcpyDeviceToHost, st));
    if (sampling) TH_HIP(hipMemcpyAsync(sp, s->s_sample, sizeof *sp, hipMemcpyDeviceToHost, st));
    TH_HIP(hipStreamSynchronize(st));
    if (poll_failures >= th::kStepReachError)
        return fail(TH_ERR_HIP, "decode: a step's context passed its chunked attention launch's chunks");
    if (poll_failures)
        return fail(TH_ERR_HIP, "decode: %u attention blocks gave up waiting for their q/k/v", poll_failures);
    return TH_OK;
}

}  // namespace

extern "C" {

int th_decode(th_model *m, th_state *s, size_t pos, size_t steps, uint32_t *out_tokens, float *out_logits) {
    return decode(m, s, pos, steps, out_tokens, out_logits, nullptr);
}

int th_decode_sample(th_model *m, th_state *s, size_t pos, size_t steps, float temperature, size_t top_k,
                     float top_p, uint64_t *rng, uint32_t *out_tokens) {
    TH_REQUIRE(rng, "th_decode_sample: null generator state");
    if (temperature == 0.0f) return decode(m, s, pos, steps, out_tokens, nullptr, nullptr);
    TH_REQUIRE(m, "th_decode_sample: null model");
    const size_t vocab = (size_t)m->c.vocab_size;
    const size_t k = std::min(std::max<size_t>(top_k, 1), vocab);
    TH_REQUIRE(k <= (size_t)th::kSampleMaxTopK, "top_k %zu: the device samples from at most %d candidates", k,
               th::kSampleMaxTopK);
    TH_REQUIRE(vocab <= th::kSampleMaxVocab, "sampling over %zu values: at most %zu", vocab, th::kSampleMaxVocab);
    TH_REQUIRE(top_p > 0.0f, "top_p must be greater than 0");
    th::SampleState ss{*rng, *rng, temperature, top_p, (int)k, 0};
    TRY(decode(m, s, pos, steps, out_tokens, nullptr, &ss));
    // The device drew once more than `steps` (the pick after the last fed
    // token, which the next call draws again): hand back the state after the
    // steps-th draw, as the reference's sampler would have it.
    *rng = steps ? ss.rng_prev : ss.rng;
    return TH_OK;
}

int th_generate(th_model *m, th_state *s, size_t pos, size_t max_tokens, const uint32_t *stop, size_t n_stop,
                float temperature, size_t top_k, float top_p, uint64_t *rng, uint32_t *out_tokens, size_t *n_out) {
    TH_REQUIRE(m && n_out, "th_generate: null argument");
    TH_NOT_CAPTURING(m->dev, "th_generate");
    *n_out = 0;
    TH_REQUIRE(n_stop >= 1 && n_stop <= (size_t)th::kStepMaxStops && stop, "th_generate: 1 to %d stop tokens",
               th::kStepMaxStops);
    for (size_t i = 0; i < n_stop; ++i)
        TH_REQUIRE(stop[i] < (uint32_t)m->c.vocab_size, "stop token %u is past the vocabulary", stop[i]);
    bool hit = false;
    if (temperature == 0.0f) return decode(m, s, pos, max_tokens, out_tokens, nullptr, nullptr, stop, n_stop, n_out, &hit);
    TH_REQUIRE(rng, "th_generate: null generator state");
    const size_t vocab = (size_t)m->c.vocab_size;
    const size_t k = std::min(std::max<size_t>(top_k, 1), vocab);
    TH_REQUIRE(k <= (size_t)th::kSampleMaxTopK, "top_k %zu: the device samples from at most %d candidates", k,
               th::kSampleMaxTopK);
    TH_REQUIRE(vocab <= th::kSampleMaxVocab, "sampling over %zu values: at most %zu", vocab, th::kSampleMaxVocab);
    TH_REQUIRE(top_p > 0.0f, "top_p must be greater than 0");
    th::SampleState ss{*rng, *rng, temperature, top_p, (int)k, 0};
    TRY(decode(m, s, pos, max_tokens, out_tokens, nullptr, &ss, stop, n_stop, n_out, &hit));
    // Ended at a stop token: every draw was used (no draw after it). Else the
    // device drew once past the last token, as in th_decode_sample.
    *rng = hit || !max_tokens ? ss.rng : ss.rng_prev;
    return TH_OK;
}

}  // extern "C"
