// Test-only entry points (include/titania_hip_test.h): each runs one fused
// kernel of the decode step or the prefill on caller buffers, so that tests
// can hold every fused kernel to the per-kernel bar against the oracle's
// composition of the reference's primitives. The product path (the Device
// entry points, th_forward, th_decode) never calls them. They allocate the
// small device state a kernel needs (step state, exchange words, bf16 hi/lo
// operands) and free it before returning.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "../../include/titania_hip_test.h"
#include "common.h"
#include "fused.h"
#include "gemm.h"
#include "step.h"

namespace {

using th::fail;

// f32 out[i] = hi[i] + lo[i] (the split_bf16 terms of a GEMM operand).
__global__ void hl_to_f32_kernel(const uint16_t *hi, const uint16_t *lo, size_t n, float *out) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        out[i] = th::bf16_to_f32(hi[i]) + th::bf16_to_f32(lo[i]);
}

// Device memory freed when the holder goes out of scope, zeroed on the
// device's stream (non-blocking, so a null-stream hipMemset would not be
// ordered before the kernels that use it).
struct DevMem {
    void *p = nullptr;
    ~DevMem() {
        if (p) (void)hipFree(p);
    }
    int alloc(size_t bytes, hipStream_t s) {
        if (hipMalloc(&p, bytes) != hipSuccess) {
            p = nullptr;
            return fail(TH_ERR_NOMEM, "test entry: %zu bytes of device memory", bytes);
        }
        if (hipMemsetAsync(p, 0, bytes, s) != hipSuccess) return fail(TH_ERR_HIP, "test entry: hipMemsetAsync failed");
        return TH_OK;
    }
};

int rows_of(const th_weight *w) { return w->ndim == 2 ? (int)w->shape[0] : 0; }
int cols_of(const th_weight *w) { return w->ndim == 2 ? (int)w->shape[1] : 0; }

}  // namespace

extern "C" {

int th_test_step_qkv(th_device *dev, const th_weight *wq, const th_weight *wk, const th_weight *wv,
                     const th_buffer *x, const th_buffer *y, const th_weight *gain, float eps, th_buffer *x_out,
                     th_buffer *qkv_out) {
    TH_REQUIRE(dev && wq && wk && wv && x && gain && x_out && qkv_out, "th_test_step_qkv: null argument");
    const int H = cols_of(wq), q_rows = rows_of(wq), kv_rows = rows_of(wk);
    TH_REQUIRE(H > 0 && cols_of(wk) == H && cols_of(wv) == H && rows_of(wv) == kv_rows, "shapes disagree");
    TH_REQUIRE(x->len == (size_t)H && (!y || y->len == (size_t)H) && x_out->len == (size_t)H &&
                   gain->numel == (size_t)H && qkv_out->len == (size_t)(q_rows + 2 * kv_rows),
               "buffer lengths disagree with the weights");
    th::StepQkvArgs q{};
    q.wq = wq->ptr;
    q.wk = wk->ptr;
    q.wv = wv->ptr;
    q.q_rows = q_rows;
    q.kv_rows = kv_rows;
    q.hidden = H;
    q.x_prev = x->ptr;
    q.y_prev = y ? y->ptr : nullptr;
    q.gain = gain->ptr;
    q.eps = eps;
    q.x_out = x_out->ptr;
    q.qkv = qkv_out->ptr;
    TH_HIP(th::launch_step_qkv(dev->stream, q));
    TH_HIP(hipStreamSynchronize(dev->stream));
    return TH_OK;
}

int th_test_step_gate_up(th_device *dev, const th_weight *gate, const th_weight *up, const th_buffer *x1,
                         const th_buffer *o, const th_weight *gain, float eps, th_buffer *x_out, th_buffer *h) {
    TH_REQUIRE(dev && gate && up && x1 && o && gain && x_out && h, "th_test_step_gate_up: null argument");
    const int I = rows_of(gate), H = cols_of(gate);
    TH_REQUIRE(I > 0 && rows_of(up) == I && cols_of(up) == H && x1->len == (size_t)H && o->len == (size_t)H &&
                   x_out->len == (size_t)H && gain->numel == (size_t)H && h->len == (size_t)I,
               "buffer lengths disagree with the weights");
    TH_HIP(th::launch_step_gate_up(dev->stream, gate->ptr, up->ptr, I, H, x1->ptr, o->ptr, gain->ptr, eps,
                                   x_out->ptr, h->ptr));
    TH_HIP(hipStreamSynchronize(dev->stream));
    return TH_OK;
}

int th_test_step_gemv(th_device *dev, const th_weight *w, const th_buffer *x, th_buffer *out) {
    TH_REQUIRE(dev && w && x && out, "th_test_step_gemv: null argument");
    const int rows = rows_of(w), cols = cols_of(w);
    TH_REQUIRE(rows > 0 && x->len == (size_t)cols && out->len == (size_t)rows,
               "buffer lengths disagree with the weight");
    TH_HIP(th::launch_step_gemv(dev->stream, w->ptr, rows, cols, x->ptr, out->ptr));
    TH_HIP(hipStreamSynchronize(dev->stream));
    return TH_OK;
}

int th_test_step_logits(th_device *dev, const th_weight *w, const th_buffer *x, const th_buffer *y,
                        const th_weight *gain, float eps, th_buffer *logits, uint32_t *token) {
    TH_REQUIRE(dev && w && x && gain && logits && token, "th_test_step_logits: null argument");
    const int V = rows_of(w), H = cols_of(w);
    TH_REQUIRE(V > 0 && x->len == (size_t)H && (!y || y->len == (size_t)H) && gain->numel == (size_t)H &&
                   logits->len == (size_t)V,
               "buffer lengths disagree with the weight");
    DevMem part, st;
    TRY(part.alloc((size_t)th::step_logits_partials(V) * sizeof(uint64_t), dev->stream));
    TRY(st.alloc(sizeof(th::StepState), dev->stream));
    int np = 0;
    TH_HIP(th::launch_step_logits(dev->stream, w->ptr, V, H, x->ptr, y ? y->ptr : nullptr, gain->ptr, eps,
                                  logits->ptr, static_cast<uint64_t *>(part.p), &np));
    TH_HIP(th::launch_pick_partials(dev->stream, static_cast<uint64_t *>(part.p), (size_t)np,
                                    static_cast<th::StepState *>(st.p), 0));
    th::StepState host{};
    TH_HIP(hipMemcpyAsync(&host, st.p, sizeof host, hipMemcpyDeviceToHost, dev->stream));
    TH_HIP(hipStreamSynchronize(dev->stream));
    *token = host.token;
    return TH_OK;
}

int th_test_step_qkv_attn(th_device *dev, const th_weight *wq, const th_weight *wk, const th_weight *wv,
                          const th_buffer *x, const th_buffer *y, const th_weight *gain, const th_weight *q_norm,
                          const th_weight *k_norm, float eps, const th_buffer *rope, th_buffer *k_cache,
                          th_buffer *v_cache, size_t max_len, size_t pos, size_t n_heads, size_t n_kv_heads,
                          th_buffer *x_out, th_buffer *att_out) {
    TH_REQUIRE(dev && wq && wk && wv && x && gain && rope && k_cache && v_cache && x_out && att_out,
               "th_test_step_qkv_attn: null argument");
    const int H = cols_of(wq);
    const size_t hd = 128, qd = n_heads * hd, kvd = n_kv_heads * hd;
    TH_REQUIRE(n_kv_heads > 0 && n_heads % n_kv_heads == 0 && (size_t)rows_of(wq) == qd &&
                   (size_t)rows_of(wk) == kvd && (size_t)rows_of(wv) == kvd && cols_of(wk) == H &&
                   cols_of(wv) == H,
               "weights are not [n_heads * 128, hidden] and [n_kv_heads * 128, hidden] x 2");
    TH_REQUIRE(x->len == (size_t)H && (!y || y->len == (size_t)H) && x_out->len == (size_t)H &&
                   gain->numel == (size_t)H && att_out->len == qd,
               "buffer lengths disagree with the weights");
    TH_REQUIRE((!q_norm || q_norm->numel == hd) && (!k_norm || k_norm->numel == hd), "q/k norms hold 128 gains");
    TH_REQUIRE(pos < max_len && rope->len >= max_len * hd, "the rope table holds max_len positions");
    // The attention blocks read whole 64-row passes: the caches extend
    // kStepKvTailRows rows of head_dim past the last head.
    const size_t need = n_kv_heads * max_len * hd + (size_t)th::kStepKvTailRows * hd;
    TH_REQUIRE(k_cache->len >= need && v_cache->len >= need, "caches need %zu floats (the tail included)", need);
    const int chunks = th::step_qkv_attn_chunks(max_len, 0, (int)n_heads);
    TH_REQUIRE(th::step_qkv_attn_supported(H, (int)n_heads, (int)n_kv_heads),
               "the fused launch does not take this shape");
    DevMem st, words, err, part;
    TRY(st.alloc(sizeof(th::StepState), dev->stream));
    const size_t nw = th::step_qkv_attn_words((int)qd, (int)kvd, (int)n_heads, std::max(chunks, 1));
    TRY(words.alloc(nw * sizeof(unsigned long long), dev->stream));
    TRY(err.alloc(sizeof(unsigned), dev->stream));
    th::StepState host{};
    host.pos = (long long)pos;
    TH_HIP(hipMemcpyAsync(st.p, &host, sizeof host, hipMemcpyHostToDevice, dev->stream));
    th::StepQkvAttnArgs f{};
    f.qkv.wq = wq->ptr;
    f.qkv.wk = wk->ptr;
    f.qkv.wv = wv->ptr;
    f.qkv.q_rows = (int)qd;
    f.qkv.kv_rows = (int)kvd;
    f.qkv.hidden = H;
    f.qkv.x_prev = x->ptr;
    f.qkv.y_prev = y ? y->ptr : nullptr;
    f.qkv.gain = gain->ptr;
    f.qkv.eps = eps;
    f.qkv.x_out = x_out->ptr;
    f.at.q_norm = q_norm ? q_norm->ptr : nullptr;
    f.at.k_norm = k_norm ? k_norm->ptr : nullptr;
    f.at.rope = rope->ptr;
    f.at.k_cache = k_cache->ptr;
    f.at.v_cache = v_cache->ptr;
    f.at.head_stride = (long long)(max_len * hd);
    f.at.pos = &static_cast<th::StepState *>(st.p)->pos;
    f.at.n_heads = (int)n_heads;
    f.at.n_kv_heads = (int)n_kv_heads;
    f.at.nsplit = 1;
    f.at.kv_bf16 = 0;
    f.at.eps = eps;
    f.at.out = att_out->ptr;
    f.words = static_cast<unsigned long long *>(words.p);
    f.err = static_cast<unsigned *>(err.p);
    f.st = static_cast<th::StepState *>(st.p);
    f.layer = 0;
    f.chunks = chunks;
    if (chunks > 0) {
        TH_HIP(th::launch_step_qkv_attn(dev->stream, f));
    } else {
        // Past the chunked launch's reach: the streaming split attention in
        // the same launch, then the combine, as the decode step runs them.
        const int nsplit = th::step_attention_splits(max_len, 0, (int)(n_heads / n_kv_heads), (int)n_kv_heads,
                                                     dev->num_cus);
        f.at.nsplit = nsplit;
        const size_t pf = th::attention_scratch(1, n_heads, hd, nsplit);
        if (pf) {
            TRY(part.alloc(pf * sizeof(float), dev->stream));
            f.at.part_acc = static_cast<float *>(part.p);
            f.at.part_ml = f.at.part_acc + n_heads * (size_t)nsplit * hd;
        }
        TH_HIP(th::launch_step_qkv_stream(dev->stream, f));
        if (nsplit > 1)
            TH_HIP(th::launch_attn_combine(dev->stream, att_out->ptr, f.at.part_acc, f.at.part_ml, n_heads, nsplit,
                                           (int)hd));
    }
    unsigned failures = 0;
    TH_HIP(hipMemcpyAsync(&failures, err.p, sizeof failures, hipMemcpyDeviceToHost, dev->stream));
    TH_HIP(hipStreamSynchronize(dev->stream));
    TH_REQUIRE(failures == 0, "%u attention blocks gave up waiting for their q/k/v", failures);
    return TH_OK;
}

int th_test_step_attention(th_device *dev, const th_buffer *qkv, const th_weight *q_norm, const th_weight *k_norm,
                           float eps, const th_buffer *rope, th_buffer *k_cache, th_buffer *v_cache, size_t max_len,
                           size_t pos, size_t n_heads, size_t n_kv_heads, int kv_bf16, th_buffer *att_out,
                           int *n_splits) {
    TH_REQUIRE(dev && qkv && rope && k_cache && v_cache && att_out, "th_test_step_attention: null argument");
    const size_t hd = 128, qd = n_heads * hd, kvd = n_kv_heads * hd;
    const size_t group = n_kv_heads ? n_heads / n_kv_heads : 0;
    TH_REQUIRE(n_kv_heads > 0 && group * n_kv_heads == n_heads && (group == 1 || group == 2 || group == 4 || group == 8),
               "the split attention takes KV groups of 1, 2, 4 or 8 q heads");
    TH_REQUIRE(qkv->len == qd + 2 * kvd && att_out->len == qd, "qkv holds the raw q, k, v rows; att_out n_heads x 128");
    TH_REQUIRE((!q_norm || q_norm->numel == hd) && (!k_norm || k_norm->numel == hd), "q/k norms hold 128 gains");
    TH_REQUIRE(kv_bf16 == 0 || kv_bf16 == 1, "kv_bf16 is 0 or 1");
    TH_REQUIRE(pos < max_len && rope->len >= max_len * hd, "the rope table holds max_len positions");
    // A pass of cached rows may start up to a pass below max_len: the caches
    // extend kStepKvTailRows rows of head_dim floats past the last head (bf16
    // caches hold two values a float).
    const size_t cache_floats = kv_bf16 ? (n_kv_heads * max_len * hd + 1) / 2 : n_kv_heads * max_len * hd;
    const size_t need = cache_floats + (size_t)th::kStepKvTailRows * hd;
    TH_REQUIRE(k_cache->len >= need && v_cache->len >= need, "caches need %zu floats (the tail included)", need);
    const int nsplit = th::step_attention_splits(max_len, kv_bf16, (int)group, (int)n_kv_heads, dev->num_cus);
    DevMem st, part;
    TRY(st.alloc(sizeof(th::StepState), dev->stream));
    th::StepState host{};
    host.pos = (long long)pos;
    TH_HIP(hipMemcpyAsync(st.p, &host, sizeof host, hipMemcpyHostToDevice, dev->stream));
    th::StepAttnArgs a{};
    a.qkv = qkv->ptr;
    a.q_norm = q_norm ? q_norm->ptr : nullptr;
    a.k_norm = k_norm ? k_norm->ptr : nullptr;
    a.rope = rope->ptr;
    a.k_cache = k_cache->ptr;
    a.v_cache = v_cache->ptr;
    a.head_stride = (long long)(max_len * hd);
    a.pos = &static_cast<th::StepState *>(st.p)->pos;
    a.n_heads = (int)n_heads;
    a.n_kv_heads = (int)n_kv_heads;
    a.nsplit = nsplit;
    a.kv_bf16 = kv_bf16;
    a.eps = eps;
    a.out = att_out->ptr;
    const size_t pf = th::attention_scratch(1, n_heads, hd, nsplit);
    if (pf) {
        TRY(part.alloc(pf * sizeof(float), dev->stream));
        a.part_acc = static_cast<float *>(part.p);
        a.part_ml = a.part_acc + n_heads * (size_t)nsplit * hd;
    }
    TH_HIP(th::launch_step_attention(dev->stream, a));
    if (nsplit > 1)
        TH_HIP(th::launch_attn_combine(dev->stream, att_out->ptr, a.part_acc, a.part_ml, n_heads, nsplit, (int)hd));
    TH_HIP(hipStreamSynchronize(dev->stream));
    if (n_splits) *n_splits = nsplit;
    return TH_OK;
}

int th_test_gemm_qkv(th_device *dev, const th_buffer *xn, const th_weight *wq, const th_weight *wk,
                     const th_weight *wv, const th_weight *q_norm, const th_weight *k_norm, float eps,
                     const th_buffer *rope, th_buffer *k_cache, th_buffer *v_cache, size_t max_len, size_t pos,
                     size_t n, size_t n_heads, size_t n_kv_heads, th_buffer *q_out, th_buffer *planes) {
    TH_REQUIRE(dev && xn && wq && wk && wv && rope && k_cache && v_cache && q_out, "th_test_gemm_qkv: null argument");
    const size_t H = (size_t)cols_of(wq), hd = 128, qd = n_heads * hd, kvd = n_kv_heads * hd;
    TH_REQUIRE(n > 0 && n_kv_heads > 0 && (size_t)rows_of(wq) == qd && (size_t)rows_of(wk) == kvd &&
                   (size_t)rows_of(wv) == kvd && (size_t)cols_of(wk) == H && (size_t)cols_of(wv) == H,
               "weights are not [n_heads * 128, hidden] and [n_kv_heads * 128, hidden] x 2");
    TH_REQUIRE(xn->len == n * H && q_out->len == n * qd, "buffer lengths disagree with n and the weights");
    TH_REQUIRE(pos + n <= max_len && rope->len >= max_len * hd, "positions past max_len or the rope table");
    TH_REQUIRE(k_cache->len >= n_kv_heads * max_len * hd && v_cache->len >= n_kv_heads * max_len * hd,
               "caches hold [n_kv_heads][max_len][128]");
    const bool head_tile = th::gemm_qkv_fused(n, qd, kvd, H, hd);
    TH_REQUIRE(head_tile || th::gemm_qkv_huge_fused(n, qd, kvd, H, hd, (long long)pos),
               "the fused q/k/v GEMM does not take this shape");
    DevMem split;
    TRY(split.alloc(2 * n * H * sizeof(uint16_t), dev->stream));
    uint16_t *hi = static_cast<uint16_t *>(split.p), *lo = hi + n * H;
    TH_HIP(th::launch_gemm_split(dev->stream, xn->ptr, n, H, hi, lo));
    th::QkvPostArgs qa{};
    qa.q = q_out->ptr;
    qa.q_norm = q_norm ? q_norm->ptr : nullptr;
    qa.k_norm = k_norm ? k_norm->ptr : nullptr;
    qa.rope = rope->ptr;
    qa.k_cache = k_cache->ptr;
    qa.v_cache = v_cache->ptr;
    qa.head_stride = (long long)(max_len * hd);
    qa.pos_stride = (long long)hd;
    qa.pos = (long long)pos;
    qa.n = (int)n;
    qa.n_heads = (int)n_heads;
    qa.n_kv_heads = (int)n_kv_heads;
    qa.head_dim = (int)hd;
    qa.kv_bf16 = 0;
    qa.eps = eps;
    if (planes) {
        const size_t bytes = th::attention_planes_bytes(max_len, n_kv_heads);
        TH_REQUIRE(planes->len * sizeof(float) >= bytes, "planes hold %zu bytes, %zu needed",
                   planes->len * sizeof(float), bytes);
        const th::PlanePtrs pp = th::attention_planes_of(planes->ptr, max_len, n_kv_heads);
        qa.kh = pp.kh;
        qa.kl = pp.kl;
        qa.vh = pp.vh;
        qa.vl = pp.vl;
        qa.plane_len = pp.plane_len;
    }
    if (head_tile)
        TH_HIP(th::launch_gemm_qkv(dev->stream, hi, lo, H, wq->ptr, wk->ptr, wv->ptr, qa));
    else
        TH_HIP(th::launch_gemm_qkv_huge(dev->stream, hi, lo, H, wq->ptr, wk->ptr, wv->ptr, qa));
    TH_HIP(hipStreamSynchronize(dev->stream));
    return TH_OK;
}

int th_test_gemm_silu(th_device *dev, const th_buffer *xn, const th_weight *gate, const th_weight *up, size_t n,
                      th_buffer *h_out) {
    TH_REQUIRE(dev && xn && gate && up && h_out, "th_test_gemm_silu: null argument");
    const size_t I = (size_t)rows_of(gate), H = (size_t)cols_of(gate);
    TH_REQUIRE(n > 0 && I > 0 && (size_t)rows_of(up) == I && (size_t)cols_of(up) == H && I % 64 == 0,
               "gate and up are not [inter, hidden] with inter a multiple of 64");
    TH_REQUIRE(xn->len == n * H && h_out->len == n * I, "buffer lengths disagree with n and the weights");
    DevMem split, hsplit;
    TRY(split.alloc(2 * n * H * sizeof(uint16_t), dev->stream));
    TRY(hsplit.alloc(2 * n * I * sizeof(uint16_t), dev->stream));
    uint16_t *hi = static_cast<uint16_t *>(split.p), *lo = hi + n * H;
    uint16_t *hh = static_cast<uint16_t *>(hsplit.p), *hl = hh + n * I;
    TH_HIP(th::launch_gemm_split(dev->stream, xn->ptr, n, H, hi, lo));
    TH_HIP(th::launch_gemm_silu(dev->stream, hi, lo, n, H, gate->ptr, up->ptr, I, hh, hl));
    hl_to_f32_kernel<<<256, 256, 0, dev->stream>>>(hh, hl, n * I, h_out->ptr);
    TH_HIP(hipGetLastError());
    TH_HIP(hipStreamSynchronize(dev->stream));
    return TH_OK;
}

int th_test_add_rmsnorm_parts(th_device *dev, th_buffer *x, const th_buffer *parts, size_t n_parts,
                              const th_weight *gain, float eps, th_buffer *xn) {
    TH_REQUIRE(dev && x && gain && xn && (parts || n_parts == 0), "th_test_add_rmsnorm_parts: null argument");
    const size_t dim = gain->numel, rows = dim ? x->len / dim : 0;
    TH_REQUIRE(dim > 0 && rows * dim == x->len && xn->len == x->len, "x and xn hold whole rows of the gains");
    TH_REQUIRE(!n_parts || parts->len == n_parts * x->len, "parts hold n_parts copies of x's length");
    DevMem split;
    TRY(split.alloc(2 * x->len * sizeof(uint16_t), dev->stream));
    uint16_t *hi = static_cast<uint16_t *>(split.p), *lo = hi + x->len;
    TH_HIP(th::launch_add_rmsnorm_parts(dev->stream, x->ptr, n_parts ? parts->ptr : nullptr, (int)n_parts, x->len,
                                        nullptr, hi, lo, rows, gain->ptr, dim, eps));
    hl_to_f32_kernel<<<256, 256, 0, dev->stream>>>(hi, lo, x->len, xn->ptr);
    TH_HIP(hipGetLastError());
    TH_HIP(hipStreamSynchronize(dev->stream));
    return TH_OK;
}

int th_test_attention_prefill(th_device *dev, const th_buffer *q, const th_buffer *k_cache, const th_buffer *v_cache,
                              size_t max_len, size_t pos, size_t n, size_t n_heads, size_t n_kv_heads, int planes,
                              th_buffer *out) {
    TH_REQUIRE(dev && q && k_cache && v_cache && out, "th_test_attention_prefill: null argument");
    const size_t hd = 128;
    TH_REQUIRE(n > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0 && pos + n <= max_len,
               "heads must split into KV groups and the tokens fit the caches");
    TH_REQUIRE(q->len == n * n_heads * hd && out->len == n * n_heads * hd, "q and out hold n x n_heads x 128");
    TH_REQUIRE(k_cache->len >= n_kv_heads * max_len * hd && v_cache->len >= n_kv_heads * max_len * hd,
               "caches hold [n_kv_heads][max_len][128]");
    th::AttnKernelArgs a{};
    a.out = out->ptr;
    a.q = q->ptr;
    a.k = k_cache->ptr;
    a.v = v_cache->ptr;
    a.n_heads = (int)n_heads;
    a.n_kv_heads = (int)n_kv_heads;
    a.group = (int)(n_heads / n_kv_heads);
    a.pos = (long long)pos;
    a.pos_stride = (long long)hd;
    a.head_stride = (long long)(max_len * hd);
    a.nsplit = th::attention_splits(n, n_heads, n_kv_heads, pos + n, hd);
    a.kv_bf16 = 0;
    a.scale = 1.0f / sqrtf((float)hd);
    DevMem part, pl;
    const size_t pf = th::attention_scratch(n, n_heads, hd, a.nsplit);
    if (pf) {
        TRY(part.alloc(pf * sizeof(float), dev->stream));
        a.part_acc = static_cast<float *>(part.p);
        a.part_ml = a.part_acc + n * n_heads * (size_t)a.nsplit * hd;
    }
    if (planes) {
        TH_REQUIRE(th::attention_planes_supported(a, n, hd), "the planes kernel does not take this shape");
        const size_t bytes = th::attention_planes_bytes(max_len, n_kv_heads);
        TRY(pl.alloc(bytes, dev->stream));
        TH_HIP(th::launch_attention_planes(dev->stream, a, n, hd, pl.p, bytes, max_len));
    } else {
        TH_HIP(th::launch_attention(dev->stream, a, n, hd));
    }
    TH_HIP(hipStreamSynchronize(dev->stream));
    return TH_OK;
}

}  // extern "C"
