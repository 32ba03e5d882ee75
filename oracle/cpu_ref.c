/*
 * CPU oracle for the Qwen3 forward pass: a C restatement of the reference
 * implementation of every `Device` operation (model/cpu.rs) and of the forward
 * pass that sequences them (model/model.rs).
 *
 * THIS IS TEST INFRASTRUCTURE. Only tests/, the smoke check and bench.py's
 * cpu_baseline leg load it, as the results to compare against or as the timed
 * CPU baseline. The product path never links, loads or falls back to it.
 *
 * Floating-point semantics follow the Rust source exactly: no FMA contraction
 * (build with -ffp-contract=off, no -ffast-math), every float sum a left fold
 * in index order, glibc expf/powf/sinf/cosf/sqrtf where Rust calls
 * f32::exp/powf/sin_cos/sqrt. Work is split across threads only where rayon
 * splits it (rows of a matmul, (token, head) pairs of attention), which cannot
 * change results because each row or head is computed sequentially.
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   ref_embed      closed form bits<<16
 *   ref_matmul     float64 brute force with a rounding bound; an independent
 *                  numpy float32 emulation of the 8-accumulator order (bit-exact)
 *   ref_rmsnorm    torch float64 rms_norm; constant-row closed form
 *   ref_rope       pos 0 identity; pair-norm preservation; HF rotate_half in float64
 *   ref_rope_table float64 closed form of theta^(-2i/d), sin/cos
 *   ref_attention  len 1 -> V row exactly; equal keys -> mean of V; float64 softmax
 *   ref_silu_mul   torch float64 silu; g = 0 -> 0
 *   ref_argmax     brute force, lowest index on ties
 *   ref_sample     temperature 0 / top_k 1 / small top_p -> the argmax; tokens
 *                  outside the top-k or the top-p prefix never drawn; draw
 *                  frequencies against the float64 softmax (chi-square); the
 *                  xorshift64* generator against a float64-free integer
 *                  restatement of its published recurrence (Vigna 2016)
 *   ref_forward    HF transformers Qwen3ForCausalLM on the same weights (fixture)
 * Unpinned at the bit level: glibc expf/powf/sinf/cosf themselves (no reference
 * test holds their outputs), which tolerance-based checks make moot.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

#define EXPORT __attribute__((visibility("default")))

static int g_threads = 0; /* 0: OpenMP default (all cores, like rayon) */

EXPORT void ref_set_threads(int n) { g_threads = n; }
EXPORT int ref_get_threads(void) { return g_threads > 0 ? g_threads : omp_get_max_threads(); }

static int nthreads(void) { return g_threads > 0 ? g_threads : omp_get_max_threads(); }

/* model/cpu.rs:158-161: bf16 is the top half of an f32. */
static inline float bf16(uint16_t bits) {
    union { uint32_t u; float f; } v;
    v.u = (uint32_t)bits << 16;
    return v.f;
}

/* model/cpu.rs:167-177: eight interleaved accumulators (mul rounded, then add),
 * folded left, plus the tail summed left. */
static inline float dot(const uint16_t *w, const float *x, size_t cols) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t done = cols / 8 * 8;
    for (size_t c = 0; c < done; c += 8) {
        for (int i = 0; i < 8; ++i) {
            float p = bf16(w[c + i]) * x[c + i];
            acc[i] = acc[i] + p;
        }
    }
    float rest = 0.0f;
    for (size_t c = done; c < cols; ++c) {
        float p = bf16(w[c]) * x[c];
        rest = rest + p;
    }
    float s = 0.0f;
    for (int i = 0; i < 8; ++i) s = s + acc[i];
    return s + rest;
}

/* model/cpu.rs:179-181 */
static inline float dot_f32(const float *a, const float *b, size_t n) {
    float s = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        float p = a[i] * b[i];
        s = s + p;
    }
    return s;
}

/* model/cpu.rs:183-193 */
static void softmax(float *x, size_t n) {
    float max = -INFINITY;
    for (size_t i = 0; i < n; ++i) max = fmaxf(max, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        x[i] = expf(x[i] - max);
        sum = sum + x[i];
    }
    for (size_t i = 0; i < n; ++i) x[i] = x[i] / sum;
}

/* model/cpu.rs:34-36 (Device::copy, model/device.rs:34-42) */
EXPORT void ref_copy(float *dst, size_t dst_offset, const float *src, size_t src_offset, size_t len) {
    memmove(dst + dst_offset, src + src_offset, len * sizeof(float));
}

/* model/cpu.rs:38-47: out[t] = table[tokens[t]], bf16 -> f32. */
EXPORT void ref_embed(float *out, const uint16_t *table, size_t dim, const uint32_t *tokens, size_t n) {
    for (size_t t = 0; t < n; ++t) {
        const uint16_t *row = table + (size_t)tokens[t] * dim;
        for (size_t i = 0; i < dim; ++i) out[t * dim + i] = bf16(row[i]);
    }
}

/* model/cpu.rs:49-77: out[t][r] = dot(w[r], x[t]); n = x_len / cols tokens.
 * The reference's n > 1 path computes the same dot per (row, token) and only
 * changes the traversal order, so both paths reduce to this loop. */
EXPORT void ref_matmul(float *out, const uint16_t *w, size_t rows, size_t cols, const float *x, size_t n) {
    long long R = (long long)rows;
#pragma omp parallel for schedule(static) num_threads(nthreads())
    for (long long r = 0; r < R; ++r) {
        const uint16_t *row = w + (size_t)r * cols;
        for (size_t t = 0; t < n; ++t) out[t * rows + (size_t)r] = dot(row, x + t * cols, cols);
    }
}

/* model/cpu.rs:79-83 */
EXPORT void ref_add(float *x, const float *y, size_t len) {
    for (size_t i = 0; i < len; ++i) x[i] = x[i] + y[i];
}

/* model/cpu.rs:85-94: each dim-long row scaled by 1/sqrt(mean square + eps),
 * the product (scale * gain) formed first. */
EXPORT void ref_rmsnorm(float *x, size_t len, const uint16_t *weight, size_t dim, float eps) {
    for (size_t r = 0; r + dim <= len; r += dim) {
        float *row = x + r;
        float ss = 0.0f;
        for (size_t i = 0; i < dim; ++i) {
            float sq = row[i] * row[i];
            ss = ss + sq;
        }
        float mean_square = ss / (float)dim;
        float scale = 1.0f / sqrtf(mean_square + eps);
        for (size_t i = 0; i < dim; ++i) {
            float g = scale * bf16(weight[i]);
            row[i] = row[i] * g;
        }
    }
}

/* model/cpu.rs:96-111: element i of each head pairs with i + head_dim/2,
 * rotated by (cos, sin) at table[((pos + t) * head_dim/2 + i) * 2]. */
EXPORT void ref_rope(float *x, size_t len, const float *table, size_t pos, size_t n_heads, size_t head_dim) {
    size_t half = head_dim / 2;
    size_t tok = n_heads * head_dim;
    for (size_t t = 0; t * tok + tok <= len; ++t) {
        const float *angles = table + (pos + t) * head_dim;
        for (size_t h = 0; h < n_heads; ++h) {
            float *head = x + t * tok + h * head_dim;
            for (size_t i = 0; i < half; ++i) {
                float c = angles[2 * i], s = angles[2 * i + 1];
                float a = head[i], b = head[i + half];
                float ac = a * c, bs = b * s, bc = b * c, as = a * s;
                head[i] = ac - bs;
                head[i + half] = bc + as;
            }
        }
    }
}

/* model/cpu.rs:113-149: causal GQA. Token t of q (position pos + t) attends
 * positions 0..=pos+t of caches laid out [position][n_kv_heads][head_dim]. */
EXPORT void ref_attention(float *out, const float *q, size_t n, const float *k_cache, const float *v_cache,
                          size_t pos, size_t n_heads, size_t head_dim, size_t n_kv_heads) {
    size_t group = n_heads / n_kv_heads;
    size_t kv_dim = n_kv_heads * head_dim;
    float scale = 1.0f / sqrtf((float)head_dim);
    long long items = (long long)(n * n_heads);
#pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads())
    for (long long it = 0; it < items; ++it) {
        size_t token = (size_t)it / n_heads, head = (size_t)it % n_heads;
        size_t len = pos + token + 1;
        size_t kv = head / group * head_dim;
        const float *qh = q + (size_t)it * head_dim;
        float *o = out + (size_t)it * head_dim;
        float *scores = (float *)malloc(len * sizeof(float));
        for (size_t t = 0; t < len; ++t) scores[t] = scale * dot_f32(qh, k_cache + t * kv_dim + kv, head_dim);
        softmax(scores, len);
        for (size_t d = 0; d < head_dim; ++d) o[d] = 0.0f;
        for (size_t t = 0; t < len; ++t) {
            const float *v = v_cache + t * kv_dim + kv;
            float p = scores[t];
            for (size_t d = 0; d < head_dim; ++d) {
                float pv = p * v[d];
                o[d] = o[d] + pv;
            }
        }
        free(scores);
    }
}

/* model/cpu.rs:151-155: g = g / (1 + exp(-g)) * u, divide first. */
EXPORT void ref_silu_mul(float *gate, const float *up, size_t len) {
    for (size_t i = 0; i < len; ++i) {
        float g = gate[i];
        float s = g / (1.0f + expf(-g));
        gate[i] = s * up[i];
    }
}

/* model/model.rs:239-250: [pos][i] = (cos, sin) of pos * theta^(-2i/head_dim). */
EXPORT void ref_rope_table(float *table, size_t max_len, size_t head_dim, float theta) {
    size_t half = head_dim / 2;
    for (size_t p = 0; p < max_len; ++p) {
        for (size_t i = 0; i < half; ++i) {
            float freq = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
            float a = (float)p * freq;
            table[(p * half + i) * 2] = cosf(a);
            table[(p * half + i) * 2 + 1] = sinf(a);
        }
    }
}

/* model/sampler.rs:21-33 at temperature 0: the largest logit under total
 * order; ties resolve to the lowest index. */
static inline int32_t total_key(float f) {
    union { float f; int32_t i; } v;
    v.f = f;
    return v.i ^ (int32_t)(((uint32_t)(v.i >> 31)) >> 1);
}

EXPORT uint32_t ref_argmax(const float *logits, size_t n) {
    size_t best = 0;
    int32_t bk = total_key(logits[0]);
    for (size_t i = 1; i < n; ++i) {
        int32_t k = total_key(logits[i]);
        if (k > bk) { bk = k; best = i; }
    }
    return (uint32_t)best;
}

/* ---- sampling (model/sampler.rs) ---- */

/* model/sampler.rs:62-76: xorshift64*; next_f32 is uniform in [0, 1). */
static uint64_t rng_next_u64(uint64_t *s) {
    uint64_t x = *s;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *s = x;
    return x * 0x2545F4914F6CDD1DULL;
}

static float rng_next_f32(uint64_t *s) { return (float)(rng_next_u64(s) >> 40) / (float)(1u << 24); }

EXPORT uint64_t ref_rng_next_u64(uint64_t *s) { return rng_next_u64(s); }

typedef struct { int32_t key; uint32_t token; } cand_t;

/* Larger logit first under total order; equal logits by lower token (the
 * reference's select_nth_unstable leaves their order unspecified). */
static int cand_cmp(const void *a, const void *b) {
    const cand_t *x = (const cand_t *)a, *y = (const cand_t *)b;
    if (x->key != y->key) return x->key > y->key ? -1 : 1;
    return x->token < y->token ? -1 : (x->token > y->token);
}

/* model/sampler.rs:21-59: the top_k largest logits (top_k clamped to
 * [1, n]), sorted; at temperature 0 the first; otherwise softmax at the
 * temperature over the k, the shortest prefix whose probability reaches
 * top_p, and a draw from the prefix with the generator in *rng. */
EXPORT uint32_t ref_sample(const float *logits, size_t n, float temperature, size_t top_k, float top_p,
                           uint64_t *rng) {
    size_t k = top_k < 1 ? 1 : (top_k > n ? n : top_k);
    cand_t *c = (cand_t *)malloc(n * sizeof(cand_t));
    for (size_t i = 0; i < n; ++i) {
        c[i].key = total_key(logits[i]);
        c[i].token = (uint32_t)i;
    }
    qsort(c, n, sizeof(cand_t), cand_cmp);
    uint32_t tok = c[0].token;
    if (temperature != 0.0f) {
        float *probs = (float *)malloc(k * sizeof(float));
        const float max = logits[c[0].token];
        for (size_t i = 0; i < k; ++i) probs[i] = expf((logits[c[i].token] - max) / temperature);
        float sum = 0.0f;
        for (size_t i = 0; i < k; ++i) sum += probs[i];
        float cumulative = 0.0f;
        size_t m = 0;
        for (size_t i = 0; i < k; ++i) {
            probs[i] /= sum;
            if (cumulative < top_p) {
                cumulative += probs[i];
                m += 1;
            }
        }
        float r = rng_next_f32(rng) * cumulative;
        tok = c[m - 1].token;
        for (size_t i = 0; i < m; ++i) {
            r -= probs[i];
            if (r <= 0.0f) {
                tok = c[i].token;
                break;
            }
        }
        free(probs);
    }
    free(c);
    return tok;
}

/* ---- the forward pass (model/model.rs:83-149, State model/model.rs:156-233) ---- */

typedef struct {
    int64_t hidden, intermediate, layers, heads, kv_heads, head_dim, vocab;
    float eps, theta;
    int64_t tied;
} ref_config;

/* Per-layer weights as raw bf16 bits, in the order model.rs:49-61 loads them.
 * q_norm / k_norm may be NULL (model.rs:55-56). */
typedef struct {
    const uint16_t *attn_norm, *q, *k, *v, *o, *q_norm, *k_norm, *mlp_norm, *gate, *up, *down;
} ref_layer;

typedef struct {
    ref_config c;
    const uint16_t *embed, *norm, *lm_head; /* lm_head NULL when tied */
    const ref_layer *layers;
} ref_model;

typedef struct {
    size_t max_len, batch;
    float *x, *xb, *q, *k, *v, *att, *gate, *up, *logits;
    float **k_cache, **v_cache;
    float *rope;
    int64_t layers;
} ref_state;

EXPORT ref_state *ref_state_new(const ref_config *c, size_t max_len, size_t batch) {
    ref_state *s = (ref_state *)calloc(1, sizeof(ref_state));
    size_t hd = (size_t)c->head_dim, qd = (size_t)(c->heads * c->head_dim), kvd = (size_t)(c->kv_heads * c->head_dim);
    s->max_len = max_len;
    s->batch = batch;
    s->layers = c->layers;
    s->x = (float *)calloc(batch * (size_t)c->hidden, 4);
    s->xb = (float *)calloc(batch * (size_t)c->hidden, 4);
    s->q = (float *)calloc(batch * qd, 4);
    s->k = (float *)calloc(batch * kvd, 4);
    s->v = (float *)calloc(batch * kvd, 4);
    s->att = (float *)calloc(batch * qd, 4);
    s->gate = (float *)calloc(batch * (size_t)c->intermediate, 4);
    s->up = (float *)calloc(batch * (size_t)c->intermediate, 4);
    s->logits = (float *)calloc((size_t)c->vocab, 4);
    s->k_cache = (float **)calloc((size_t)c->layers, sizeof(float *));
    s->v_cache = (float **)calloc((size_t)c->layers, sizeof(float *));
    for (int64_t l = 0; l < c->layers; ++l) {
        s->k_cache[l] = (float *)calloc(max_len * kvd, 4);
        s->v_cache[l] = (float *)calloc(max_len * kvd, 4);
    }
    s->rope = (float *)malloc(max_len * hd * 4);
    ref_rope_table(s->rope, max_len, hd, c->theta);
    return s;
}

EXPORT void ref_state_free(ref_state *s) {
    if (!s) return;
    free(s->x); free(s->xb); free(s->q); free(s->k); free(s->v); free(s->att);
    free(s->gate); free(s->up); free(s->logits);
    for (int64_t l = 0; l < s->layers; ++l) { free(s->k_cache[l]); free(s->v_cache[l]); }
    free(s->k_cache); free(s->v_cache); free(s->rope); free(s);
}

/* Read access to a layer's caches ([max_len][kv_heads][head_dim] f32), for checks. */
EXPORT const float *ref_state_k_cache(const ref_state *s, int64_t layer) { return s->k_cache[layer]; }
EXPORT const float *ref_state_v_cache(const ref_state *s, int64_t layer) { return s->v_cache[layer]; }

/* model/model.rs:93-149 for one batch of n tokens at position pos. */
static void forward_batch(const ref_model *m, ref_state *s, const uint32_t *tokens, size_t n, size_t pos) {
    const ref_config *c = &m->c;
    size_t H = (size_t)c->hidden, I = (size_t)c->intermediate, hd = (size_t)c->head_dim;
    size_t nh = (size_t)c->heads, nkv = (size_t)c->kv_heads;
    size_t qd = nh * hd, kvd = nkv * hd;
    float eps = c->eps;

    ref_embed(s->x, m->embed, H, tokens, n);
    for (int64_t i = 0; i < c->layers; ++i) {
        const ref_layer *L = &m->layers[i];
        ref_copy(s->xb, 0, s->x, 0, n * H);
        ref_rmsnorm(s->xb, n * H, L->attn_norm, H, eps);
        ref_matmul(s->q, L->q, qd, H, s->xb, n);
        ref_matmul(s->k, L->k, kvd, H, s->xb, n);
        ref_matmul(s->v, L->v, kvd, H, s->xb, n);
        if (L->q_norm) ref_rmsnorm(s->q, n * qd, L->q_norm, hd, eps);
        if (L->k_norm) ref_rmsnorm(s->k, n * kvd, L->k_norm, hd, eps);
        ref_rope(s->q, n * qd, s->rope, pos, nh, hd);
        ref_rope(s->k, n * kvd, s->rope, pos, nkv, hd);
        ref_copy(s->k_cache[i], pos * kvd, s->k, 0, n * kvd);
        ref_copy(s->v_cache[i], pos * kvd, s->v, 0, n * kvd);
        ref_attention(s->att, s->q, n, s->k_cache[i], s->v_cache[i], pos, nh, hd, nkv);
        ref_matmul(s->xb, L->o, H, qd, s->att, n);
        ref_add(s->x, s->xb, n * H);

        ref_copy(s->xb, 0, s->x, 0, n * H);
        ref_rmsnorm(s->xb, n * H, L->mlp_norm, H, eps);
        ref_matmul(s->gate, L->gate, I, H, s->xb, n);
        ref_matmul(s->up, L->up, I, H, s->xb, n);
        ref_silu_mul(s->gate, s->up, n * I);
        ref_matmul(s->xb, L->down, H, I, s->gate, n);
        ref_add(s->x, s->xb, n * H);
    }
    ref_copy(s->xb, 0, s->x, (n - 1) * H, H);
    ref_rmsnorm(s->xb, H, m->norm, H, eps);
    ref_matmul(s->logits, m->lm_head ? m->lm_head : m->embed, (size_t)c->vocab, H, s->xb, 1);
}

/* model/model.rs:83-91: runs tokens in chunks of at most `batch` (BATCH = 64 in
 * the reference; results do not depend on the chunking) and leaves the logits
 * of the token after the last in logits_out. Returns 0, or -1 on misuse. */
EXPORT int ref_forward(const ref_model *m, ref_state *s, const uint32_t *tokens, size_t n, size_t pos,
                       float *logits_out) {
    if (n == 0 || pos + n > s->max_len) return -1;
    for (size_t i = 0; i < n; i += s->batch) {
        size_t b = n - i < s->batch ? n - i : s->batch;
        forward_batch(m, s, tokens + i, b, pos + i);
    }
    if (logits_out) memcpy(logits_out, s->logits, (size_t)m->c.vocab * sizeof(float));
    return 0;
}

/* Greedy generation as Chat::generate drives it at temperature 0
 * (model/chat.rs:142-178, model/sampler.rs:21-33): feed the prompt, then
 * `steps` times pick the argmax and feed it back; every picked token is fed,
 * the last one included (model/chat.rs:170-172), so this runs `steps`
 * single-token forward passes. out_tokens gets the `steps` tokens. If
 * top2_gaps is not NULL it gets, per step, the gap between the two largest
 * logits the token was picked from, which bounds how much error a device may
 * make before its greedy choice could differ. last_logits gets the logits
 * after the last token fed. */
EXPORT int ref_generate(const ref_model *m, ref_state *s, const uint32_t *prompt, size_t n_prompt, size_t steps,
                        uint32_t *out_tokens, float *top2_gaps, float *last_logits) {
    size_t V = (size_t)m->c.vocab;
    if (ref_forward(m, s, prompt, n_prompt, 0, NULL) != 0) return -1;
    size_t pos = n_prompt;
    for (size_t i = 0; i < steps; ++i) {
        uint32_t tok = ref_argmax(s->logits, V);
        out_tokens[i] = tok;
        if (top2_gaps) {
            float best = s->logits[tok], second = -INFINITY;
            for (size_t j = 0; j < V; ++j)
                if (j != tok && s->logits[j] > second) second = s->logits[j];
            top2_gaps[i] = best - second;
        }
        if (ref_forward(m, s, &tok, 1, pos, NULL) != 0) return -1;
        pos += 1;
    }
    if (last_logits) memcpy(last_logits, s->logits, V * sizeof(float));
    return 0;
}

/* model/chat.rs:149-178 with a Sampler (model/sampler.rs): the prompt, then
 * `steps` tokens each drawn from the logits of the token before. */
EXPORT int ref_generate_sampled(const ref_model *m, ref_state *s, const uint32_t *prompt, size_t n_prompt,
                                size_t steps, float temperature, size_t top_k, float top_p, uint64_t *rng,
                                uint32_t *out_tokens) {
    size_t V = (size_t)m->c.vocab;
    if (ref_forward(m, s, prompt, n_prompt, 0, NULL) != 0) return -1;
    size_t pos = n_prompt;
    for (size_t i = 0; i < steps; ++i) {
        uint32_t tok = ref_sample(s->logits, V, temperature, top_k, top_p, rng);
        out_tokens[i] = tok;
        if (ref_forward(m, s, &tok, 1, pos, NULL) != 0) return -1;
        pos += 1;
    }
    return 0;
}
