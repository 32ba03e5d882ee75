// The C ABI of the hip device: one entry point per method of the reference's
// Device trait (model/device.rs:9-89), argument checks mirroring the
// reference's asserts, and the fused extensions.
#include <cstdint>
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>

#include "common.h"
#include "gemm.h"
#include "sample.h"
#include "step.h"

namespace {
thread_local std::string g_error;
}

namespace th {

int fail(int code, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

void clear_error() { g_error.clear(); }

void *scratch(th_device *dev, size_t bytes) {
    if (bytes <= dev->scratch_bytes) return dev->scratch;
    if (dev->capturing) {  // growing it would wait for the stream and allocate
        fail(TH_ERR_INVALID, "%zu bytes of device scratch: more than it held when the capture began", bytes);
        return nullptr;
    }
    size_t want = std::max(bytes, dev->scratch_bytes * 2);
    want = (want + 255) & ~(size_t)255;
    if (dev->scratch) {
        if (hipStreamSynchronize(dev->stream) != hipSuccess) return nullptr;
        (void)hipFree(dev->scratch);
        dev->scratch = nullptr;
        dev->scratch_bytes = 0;
    }
    if (hipMalloc(&dev->scratch, want) != hipSuccess) {
        dev->scratch = nullptr;
        return nullptr;
    }
    dev->scratch_bytes = want;
    return dev->scratch;
}

// Copies host token ids into the device's staging area, checking each against
// the table's row count (the reference indexes out of bounds and panics).
static int stage_tokens(th_device *dev, const uint32_t *tokens, size_t n, size_t limit, uint32_t **out) {
    for (size_t i = 0; i < n; ++i)
        TH_REQUIRE(tokens[i] < limit, "token %u at index %zu is past the table's %zu rows", tokens[i], i, limit);
    if (n > dev->tokens_cap) {
        size_t cap = std::max<size_t>(n, 1024);
        uint32_t *p = nullptr;
        TH_HIP(hipStreamSynchronize(dev->stream));
        if (dev->tokens) TH_HIP(hipFree(dev->tokens));
        dev->tokens = nullptr;
        dev->tokens_cap = 0;
        TH_HIP(hipMalloc(&p, cap * sizeof(uint32_t)));
        dev->tokens = p;
        dev->tokens_cap = cap;
    }
    TH_HIP(hipMemcpyAsync(dev->tokens, tokens, n * sizeof(uint32_t), hipMemcpyHostToDevice, dev->stream));
    *out = dev->tokens;
    return TH_OK;
}

}  // namespace th

using th::fail;

extern "C" {

const char *th_last_error(void) { return g_error.c_str(); }

int th_device_create(int ordinal, th_device **out) {
    th::clear_error();
    TH_REQUIRE(out != nullptr, "th_device_create: null output");
    int count = 0;
    TH_HIP(hipGetDeviceCount(&count));
    TH_REQUIRE(ordinal >= 0 && ordinal < count, "no GPU %d (%d present)", ordinal, count);
    TH_HIP(hipSetDevice(ordinal));
    hipDeviceProp_t prop;
    TH_HIP(hipGetDeviceProperties(&prop, ordinal));
    auto *dev = new (std::nothrow) th_device();
    if (!dev) return fail(TH_ERR_NOMEM, "out of host memory");
    dev->ordinal = ordinal;
    dev->num_cus = prop.multiProcessorCount;
    if (th::noalloc_scratch_address(&dev->noalloc_scratch) != TH_OK) {  // the message is set
        delete dev;
        return TH_ERR_HIP;
    }
    hipError_t e = hipStreamCreateWithFlags(&dev->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipMalloc(&dev->token_out, 256);
    if (e == hipSuccess) e = hipEventCreate(&dev->ev_begin);
    if (e == hipSuccess) e = hipEventCreate(&dev->ev_end);
    if (e != hipSuccess) {
        th_device_destroy(dev);
        return fail(TH_ERR_HIP, "device setup failed: %s", hipGetErrorString(e));
    }
    *out = dev;
    return TH_OK;
}

void th_device_destroy(th_device *dev) {
    if (!dev) return;
    (void)hipSetDevice(dev->ordinal);
    if (dev->capturing) {  // an open capture is discarded
        hipGraph_t g = nullptr;
        if (hipStreamEndCapture(dev->stream, &g) == hipSuccess && g) (void)hipGraphDestroy(g);
        dev->capturing = false;
    }
    if (dev->stream) (void)hipStreamSynchronize(dev->stream);
    if (dev->tokens) (void)hipFree(dev->tokens);
    if (dev->scratch) (void)hipFree(dev->scratch);
    if (dev->token_out) (void)hipFree(dev->token_out);
    if (dev->ev_begin) (void)hipEventDestroy(dev->ev_begin);
    if (dev->ev_end) (void)hipEventDestroy(dev->ev_end);
    if (dev->stream) (void)hipStreamDestroy(dev->stream);
    delete dev;
}

struct th_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

int th_graph_begin(th_device *dev) {
    TH_REQUIRE(dev, "th_graph_begin: null device");
    TH_REQUIRE(!dev->capturing, "the device's stream is already being captured");
    TH_HIP(hipSetDevice(dev->ordinal));
    TH_HIP(hipStreamBeginCapture(dev->stream, hipStreamCaptureModeThreadLocal));
    dev->capturing = true;
    return TH_OK;
}

int th_graph_end(th_device *dev, th_graph **out) {
    TH_REQUIRE(dev && out, "th_graph_end: null argument");
    TH_REQUIRE(dev->capturing, "th_graph_end without th_graph_begin");
    dev->capturing = false;
    hipGraph_t graph = nullptr;
    TH_HIP(hipStreamEndCapture(dev->stream, &graph));
    auto *g = new (std::nothrow) th_graph();
    if (!g) {
        (void)hipGraphDestroy(graph);
        return fail(TH_ERR_NOMEM, "out of host memory");
    }
    g->graph = graph;
    const hipError_t e = hipGraphInstantiate(&g->exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        delete g;
        return fail(TH_ERR_HIP, "hipGraphInstantiate failed: %s", hipGetErrorString(e));
    }
    *out = g;
    return TH_OK;
}

int th_graph_launch(th_device *dev, const th_graph *g) {
    TH_REQUIRE(dev && g, "th_graph_launch: null argument");
    TH_NOT_CAPTURING(dev, "th_graph_launch");
    TH_HIP(hipGraphLaunch(g->exec, dev->stream));
    return TH_OK;
}

void th_graph_free(th_device *dev, th_graph *g) {
    if (!g) return;
    if (dev && dev->capturing) {
        th::fail(TH_ERR_INVALID, "th_graph_free cannot run while the device's stream is being captured");
        return;
    }
    if (dev) (void)hipStreamSynchronize(dev->stream);
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
}

int th_device_synchronize(th_device *dev) {
    TH_REQUIRE(dev, "null device");
    TH_NOT_CAPTURING(dev, "th_device_synchronize");
    TH_HIP(hipStreamSynchronize(dev->stream));
    return TH_OK;
}

int th_timer_begin(th_device *dev) {
    TH_REQUIRE(dev, "null device");
    TH_NOT_CAPTURING(dev, "th_timer_begin");
    TH_HIP(hipEventRecord(dev->ev_begin, dev->stream));
    return TH_OK;
}

int th_timer_end(th_device *dev, float *ms) {
    TH_REQUIRE(dev && ms, "th_timer_end: null argument");
    TH_NOT_CAPTURING(dev, "th_timer_end");
    TH_HIP(hipEventRecord(dev->ev_end, dev->stream));
    TH_HIP(hipEventSynchronize(dev->ev_end));
    TH_HIP(hipEventElapsedTime(ms, dev->ev_begin, dev->ev_end));
    return TH_OK;
}

int th_upload(th_device *dev, const uint16_t *data, const size_t *shape, size_t ndim, th_weight **out) {
    TH_REQUIRE(dev && shape && out, "th_upload: null argument");
    TH_NOT_CAPTURING(dev, "th_upload");
    TH_REQUIRE(ndim == 1 || ndim == 2, "a weight has 1 or 2 dimensions, not %zu", ndim);
    size_t numel = 1;
    for (size_t i = 0; i < ndim; ++i)
        TH_REQUIRE(!__builtin_mul_overflow(numel, shape[i], &numel) && numel <= SIZE_MAX / 2,
                   "th_upload: the element count of the shape overflows");
    TH_REQUIRE(numel == 0 || data, "th_upload: null data");
    auto *w = new (std::nothrow) th_weight();
    if (!w) return fail(TH_ERR_NOMEM, "out of host memory");
    w->ndim = ndim;
    w->shape[0] = shape[0];
    w->shape[1] = ndim == 2 ? shape[1] : 0;
    w->numel = numel;
    size_t bytes = std::max<size_t>(numel * 2, 16);
    hipError_t e = hipMalloc(&w->ptr, bytes);
    if (e == hipSuccess && numel) e = hipMemcpyAsync(w->ptr, data, numel * 2, hipMemcpyHostToDevice, dev->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(dev->stream);
    if (e != hipSuccess) {
        if (w->ptr) (void)hipFree(w->ptr);
        delete w;
        return fail(e == hipErrorOutOfMemory ? TH_ERR_NOMEM : TH_ERR_HIP, "upload of %zu bf16 failed: %s", numel,
                    hipGetErrorString(e));
    }
    *out = w;
    return TH_OK;
}

void th_weight_free(th_device *dev, th_weight *w) {
    if (!w) return;
    if (dev && dev->capturing) {  // the handle stays valid: free it after th_graph_end
        th::fail(TH_ERR_INVALID, "th_weight_free cannot run while the device's stream is being captured");
        return;
    }
    if (dev) (void)hipStreamSynchronize(dev->stream);
    if (w->ptr) (void)hipFree(w->ptr);
    delete w;
}

int th_weight_shape(const th_weight *w, size_t *shape, size_t *ndim) {
    TH_REQUIRE(w && shape && ndim, "th_weight_shape: null argument");
    *ndim = w->ndim;
    shape[0] = w->shape[0];
    if (w->ndim == 2) shape[1] = w->shape[1];
    return TH_OK;
}

int th_alloc(th_device *dev, size_t len, th_buffer **out) {
    TH_REQUIRE(dev && out, "th_alloc: null argument");
    TH_NOT_CAPTURING(dev, "th_alloc");
    auto *b = new (std::nothrow) th_buffer();
    if (!b) return fail(TH_ERR_NOMEM, "out of host memory");
    size_t bytes = std::max<size_t>(len * sizeof(float), 16);
    hipError_t e = hipMalloc(&b->ptr, bytes);
    if (e == hipSuccess) e = hipMemsetAsync(b->ptr, 0, bytes, dev->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(dev->stream);
    if (e != hipSuccess) {
        if (b->ptr) (void)hipFree(b->ptr);
        delete b;
        return fail(e == hipErrorOutOfMemory ? TH_ERR_NOMEM : TH_ERR_HIP, "alloc of %zu floats failed: %s", len,
                    hipGetErrorString(e));
    }
    b->len = b->cap = len;
    *out = b;
    return TH_OK;
}

void th_buffer_free(th_device *dev, th_buffer *b) {
    if (!b) return;
    if (dev && dev->capturing) {  // the handle stays valid: free it after th_graph_end
        th::fail(TH_ERR_INVALID, "th_buffer_free cannot run while the device's stream is being captured");
        return;
    }
    if (dev) (void)hipStreamSynchronize(dev->stream);
    if (b->ptr) (void)hipFree(b->ptr);
    delete b;
}

// model/cpu.rs:22 / model/titania.rs:125
int th_resize(th_device *dev, th_buffer *b, size_t len) {
    TH_REQUIRE(dev && b, "th_resize: null argument");
    TH_REQUIRE(len <= b->cap, "a buffer of %zu activations can't hold %zu", b->cap, len);
    b->len = len;
    return TH_OK;
}

size_t th_buffer_len(const th_buffer *b) { return b ? b->len : 0; }

int th_read(th_device *dev, const th_buffer *b, float *out, size_t len) {
    TH_REQUIRE(dev && b, "th_read: null argument");
    TH_NOT_CAPTURING(dev, "th_read");
    TH_REQUIRE(len == b->len, "reading %zu activations from a buffer of %zu", len, b->len);
    TH_REQUIRE(len == 0 || out, "th_read: null output");
    if (len) TH_HIP(hipMemcpyAsync(out, b->ptr, len * sizeof(float), hipMemcpyDeviceToHost, dev->stream));
    TH_HIP(hipStreamSynchronize(dev->stream));
    return TH_OK;
}

// model/titania.rs:133-137: data.len must equal the buffer's length.
int th_write(th_device *dev, th_buffer *b, const float *data, size_t len) {
    TH_REQUIRE(dev && b, "th_write: null argument");
    TH_NOT_CAPTURING(dev, "th_write");
    TH_REQUIRE(len == b->len, "writing %zu activations into a buffer of %zu", len, b->len);
    TH_REQUIRE(len == 0 || data, "th_write: null data");
    if (len) TH_HIP(hipMemcpyAsync(b->ptr, data, len * sizeof(float), hipMemcpyHostToDevice, dev->stream));
    TH_HIP(hipStreamSynchronize(dev->stream));
    return TH_OK;
}

// model/titania.rs:139-143
int th_copy(th_device *dev, th_buffer *dst, size_t dst_offset, const th_buffer *src, size_t src_offset,
            size_t len) {
    TH_REQUIRE(dev && dst && src, "th_copy: null argument");
    TH_REQUIRE(dst_offset <= dst->len && len <= dst->len - dst_offset, "copy of %zu to offset %zu of a buffer of %zu",
               len, dst_offset, dst->len);
    TH_REQUIRE(src_offset <= src->len && len <= src->len - src_offset,
               "copy of %zu from offset %zu of a buffer of %zu", len, src_offset, src->len);
    TH_HIP(th::launch_copy(dev->stream, dst->ptr + dst_offset, src->ptr + src_offset, len));
    return TH_OK;
}

// model/cpu.rs:38-47 / model/titania.rs:145-151
int th_embed(th_device *dev, th_buffer *out, const th_weight *table, const uint32_t *tokens, size_t n) {
    TH_REQUIRE(dev && out && table, "th_embed: null argument");
    TH_NOT_CAPTURING(dev, "th_embed");
    TH_REQUIRE(table->ndim == 2, "an embedding table has 2 dimensions");
    size_t dim = table->shape[1];
    TH_REQUIRE(out->len == n * dim, "embedding %zu tokens of %zu into a buffer of %zu", n, dim, out->len);
    if (n == 0) return TH_OK;
    TH_REQUIRE(tokens, "th_embed: null tokens");
    uint32_t *d_tokens = nullptr;
    int rc = th::stage_tokens(dev, tokens, n, table->shape[0], &d_tokens);
    if (rc != TH_OK) return rc;
    TH_HIP(th::launch_embed(dev->stream, out->ptr, table->ptr, dim, d_tokens, n));
    return TH_OK;
}

// model/cpu.rs:49-53 / model/titania.rs:153-157
int th_matmul(th_device *dev, th_buffer *out, const th_weight *w, const th_buffer *x) {
    TH_REQUIRE(dev && out && w && x, "th_matmul: null argument");
    TH_REQUIRE(w->ndim == 2, "a matmul weight has 2 dimensions");
    size_t rows = w->shape[0], cols = w->shape[1];
    TH_REQUIRE(cols > 0, "a matmul weight has columns");
    size_t n = x->len / cols;
    TH_REQUIRE(x->len == n * cols, "x holds %zu activations, not a whole number of %zu-long rows", x->len, cols);
    TH_REQUIRE(out->len == n * rows, "out holds %zu activations, not %zu tokens x %zu rows", out->len, n, rows);
    TH_REQUIRE(out->ptr != x->ptr || n == 0, "matmul cannot write its input");
    if (n >= th::kGemmMinTokens && th::gemm_supported(rows, cols))
        TH_NOT_CAPTURING(dev, "a matmul of 16 or more tokens (stream-ordered scratch)");
    // One token: the decode step's GEMV (every row's loads in flight before
    // the input is read) where it takes the row length.
    if (n == 1 && th::step_gemv_supported((int)cols) && rows < ((size_t)1 << 30))
        TH_HIP(th::launch_step_gemv(dev->stream, w->ptr, (int)rows, (int)cols, x->ptr, out->ptr));
    else
        TH_HIP(th::launch_matmul(dev->stream, out->ptr, w->ptr, rows, cols, x->ptr, n));
    return TH_OK;
}

// model/cpu.rs:79-83 (zip: the shorter length)
int th_add(th_device *dev, th_buffer *x, const th_buffer *y) {
    TH_REQUIRE(dev && x && y, "th_add: null argument");
    TH_HIP(th::launch_add(dev->stream, x->ptr, y->ptr, std::min(x->len, y->len)));
    return TH_OK;
}

// model/cpu.rs:85-94: whole weight.len-long rows.
int th_rmsnorm(th_device *dev, th_buffer *x, const th_weight *w, float eps) {
    TH_REQUIRE(dev && x && w, "th_rmsnorm: null argument");
    size_t dim = w->numel;
    TH_REQUIRE(dim > 0, "an rmsnorm weight has elements");
    TH_HIP(th::launch_rmsnorm(dev->stream, x->ptr, x->len / dim, w->ptr, dim, eps));
    return TH_OK;
}

// model/cpu.rs:96-111 / model/titania.rs:177-184
int th_rope(th_device *dev, th_buffer *x, const th_buffer *table, size_t pos, size_t n_heads, size_t head_dim) {
    TH_REQUIRE(dev && x && table, "th_rope: null argument");
    TH_REQUIRE(n_heads > 0 && head_dim > 0 && head_dim % 2 == 0, "rope needs heads of an even length");
    size_t n = x->len / (n_heads * head_dim);
    TH_REQUIRE(x->len == n * n_heads * head_dim, "x holds %zu activations, not whole tokens of %zu x %zu", x->len,
               n_heads, head_dim);
    if (n == 0) return TH_OK;
    TH_REQUIRE((pos + n) * head_dim <= table->len, "position %zu is past the end of the table", pos + n - 1);
    TH_HIP(th::launch_rope(dev->stream, x->ptr, n, table->ptr, pos, n_heads, head_dim));
    return TH_OK;
}

}  // extern "C"

namespace {

// th_attention (model/cpu.rs:113-149 / model/titania.rs:186-209), with its
// split partials in the device's growable scratch, or (fixed) in the no-alloc
// array, refusing calls whose partials outgrow it.
int attention(th_device *dev, th_buffer *out, const th_buffer *q, const th_buffer *k_cache, const th_buffer *v_cache,
              size_t pos, size_t n_heads, size_t head_dim, size_t n_kv_heads, bool fixed) {
    TH_REQUIRE(dev && out && q && k_cache && v_cache, "th_attention: null argument");
    TH_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
               "%zu query heads do not split into groups over %zu KV heads", n_heads, n_kv_heads);
    TH_REQUIRE(n_heads / n_kv_heads <= 8, "at most 8 query heads per KV head are supported");
    TH_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256, "head_dim %zu is not 64, 128 or 256",
               head_dim);
    size_t n = q->len / (n_heads * head_dim);
    TH_REQUIRE(q->len == n * n_heads * head_dim, "q holds %zu activations, not whole tokens", q->len);
    TH_REQUIRE(out->len == q->len, "out holds %zu activations, q %zu", out->len, q->len);
    if (n == 0) return TH_OK;
    size_t kv_dim = n_kv_heads * head_dim;
    TH_REQUIRE(k_cache->len >= (pos + n) * kv_dim && v_cache->len >= (pos + n) * kv_dim,
               "the caches do not hold position %zu", pos + n - 1);
    TH_REQUIRE(out->ptr != q->ptr, "attention cannot write its queries");
    int nsplit = th::attention_splits(n, n_heads, n_kv_heads, pos + n, head_dim);
    size_t floats = th::attention_scratch(n, n_heads, head_dim, nsplit);
    float *scr = nullptr;
    if (floats && fixed) {
        TH_REQUIRE(floats * sizeof(float) <= th::noalloc_scratch_bytes(),
                   "th_attention_noalloc: %zu bytes of split partials exceed its fixed %zu-byte scratch",
                   floats * sizeof(float), th::noalloc_scratch_bytes());
        scr = static_cast<float *>(dev->noalloc_scratch);
    } else if (floats) {
        scr = static_cast<float *>(th::scratch(dev, floats * sizeof(float)));
        if (!scr) return fail(TH_ERR_NOMEM, "no scratch for attention (%zu floats)", floats);
    }
    th::AttnKernelArgs a{};
    a.out = out->ptr;
    a.q = q->ptr;
    a.k = k_cache->ptr;
    a.v = v_cache->ptr;
    a.n_heads = (int)n_heads;
    a.n_kv_heads = (int)n_kv_heads;
    a.group = (int)(n_heads / n_kv_heads);
    a.pos = (long long)pos;
    a.pos_dev = nullptr;
    a.pos_stride = (long long)kv_dim;  // reference layout: [position][kv head][head_dim]
    a.head_stride = (long long)head_dim;
    a.nsplit = nsplit;
    a.kv_bf16 = 0;
    a.scale = 1.0f / sqrtf((float)head_dim);
    a.part_acc = scr;
    a.part_ml = scr ? scr + n * n_heads * (size_t)nsplit * head_dim : nullptr;
    TH_HIP(th::launch_attention(dev->stream, a, n, head_dim));
    return TH_OK;
}

}  // namespace

extern "C" {

int th_attention(th_device *dev, th_buffer *out, const th_buffer *q, const th_buffer *k_cache,
                 const th_buffer *v_cache, size_t pos, size_t n_heads, size_t head_dim, size_t n_kv_heads) {
    return attention(dev, out, q, k_cache, v_cache, pos, n_heads, head_dim, n_kv_heads, false);
}

int th_attention_noalloc(th_device *dev, th_buffer *out, const th_buffer *q, const th_buffer *k_cache,
                         const th_buffer *v_cache, size_t pos, size_t n_heads, size_t head_dim, size_t n_kv_heads) {
    return attention(dev, out, q, k_cache, v_cache, pos, n_heads, head_dim, n_kv_heads, true);
}

// model/cpu.rs:151-155 (zip: the shorter length)
int th_silu_mul(th_device *dev, th_buffer *gate, const th_buffer *up) {
    TH_REQUIRE(dev && gate && up, "th_silu_mul: null argument");
    TH_HIP(th::launch_silu_mul(dev->stream, gate->ptr, up->ptr, std::min(gate->len, up->len)));
    return TH_OK;
}

int th_add_rmsnorm(th_device *dev, th_buffer *x, const th_buffer *y, th_buffer *xb, const th_weight *w,
                   float eps) {
    TH_REQUIRE(dev && x && xb && w, "th_add_rmsnorm: null argument");
    size_t dim = w->numel;
    TH_REQUIRE(dim > 0, "an rmsnorm weight has elements");
    TH_REQUIRE(xb->len == x->len, "xb holds %zu activations, x %zu", xb->len, x->len);
    TH_REQUIRE(!y || y->len >= x->len, "y holds %zu activations, x %zu", y ? y->len : 0, x->len);
    // y may be xb: each row of y is read before that row of xb is written.
    TH_REQUIRE(!y || y->ptr != x->ptr, "y must not alias x");
    TH_HIP(th::launch_add_rmsnorm(dev->stream, x->ptr, y ? y->ptr : nullptr, xb->ptr, x->len / dim, w->ptr, dim,
                                  eps));
    return TH_OK;
}

int th_qkv_rope_append(th_device *dev, th_buffer *q, th_buffer *k, th_buffer *v, const th_weight *wq,
                       const th_weight *wk, const th_weight *wv, const th_weight *q_norm, const th_weight *k_norm,
                       const th_buffer *xb, const th_buffer *rope, th_buffer *k_cache, th_buffer *v_cache, size_t pos,
                       size_t n_heads, size_t n_kv_heads, size_t head_dim, float eps) {
    TH_REQUIRE(dev && q && k && v && wq && wk && wv && xb && rope && k_cache && v_cache,
               "th_qkv_rope_append: null argument");
    TH_REQUIRE(n_heads > 0 && n_kv_heads > 0 && head_dim > 0 && head_dim % 2 == 0 && head_dim <= 512,
               "heads of an even head_dim of at most 512");
    const size_t qd = n_heads * head_dim, kvd = n_kv_heads * head_dim;
    TH_REQUIRE(wq->ndim == 2 && wk->ndim == 2 && wv->ndim == 2 && wq->shape[0] == qd && wk->shape[0] == kvd &&
                   wv->shape[0] == kvd && wq->shape[1] > 0 && wk->shape[1] == wq->shape[1] &&
                   wv->shape[1] == wq->shape[1],
               "weights are not [n_heads * head_dim, hidden] and [n_kv_heads * head_dim, hidden] x 2");
    const size_t H = wq->shape[1], n = xb->len / H;
    TH_REQUIRE(n > 0 && xb->len == n * H, "xb holds %zu activations, not whole rows of %zu", xb->len, H);
    TH_REQUIRE(q->len == n * qd && k->len == n * kvd && v->len == n * kvd,
               "q, k and v hold %zu tokens of n_heads and n_kv_heads heads", n);
    TH_REQUIRE(q->ptr != xb->ptr && k->ptr != xb->ptr && v->ptr != xb->ptr, "q, k and v cannot be xb");
    TH_REQUIRE((!q_norm || q_norm->numel == head_dim) && (!k_norm || k_norm->numel == head_dim),
               "q/k norms hold head_dim gains");
    TH_REQUIRE((pos + n) * head_dim <= rope->len, "position %zu is past the end of the table", pos + n - 1);
    TH_REQUIRE((pos + n) * kvd <= k_cache->len && (pos + n) * kvd <= v_cache->len,
               "tokens past the end of the caches");
    // The projections (model.rs:108-110): one GEMV launch for all three rows
    // sets at one token, one matrix-core GEMM from 16 tokens.
    if (n == 1 && th::step_gemv_supported((int)H)) {
        const uint16_t *w[3] = {wq->ptr, wk->ptr, wv->ptr};
        const int rows[3] = {(int)qd, (int)kvd, (int)kvd};
        float *const out[3] = {q->ptr, k->ptr, v->ptr};
        TH_HIP(th::launch_step_gemv3(dev->stream, w, rows, (int)H, xb->ptr, out));
    } else if (n >= th::kGemmMinTokens && th::gemm_supported(qd, H) && th::gemm_supported(kvd, H)) {
        TH_NOT_CAPTURING(dev, "a projection of 16 or more tokens (stream-ordered scratch)");
        const th::GemmOut o[3] = {{wq->ptr, qd, q->ptr}, {wk->ptr, kvd, k->ptr}, {wv->ptr, kvd, v->ptr}};
        TH_HIP(th::launch_gemm_outs(dev->stream, xb->ptr, n, H, o, 3));
    } else {
        if (n >= th::kGemmMinTokens) TH_NOT_CAPTURING(dev, "a projection of 16 or more tokens (stream-ordered scratch)");
        TH_HIP(th::launch_matmul(dev->stream, q->ptr, wq->ptr, qd, H, xb->ptr, n));
        TH_HIP(th::launch_matmul(dev->stream, k->ptr, wk->ptr, kvd, H, xb->ptr, n));
        TH_HIP(th::launch_matmul(dev->stream, v->ptr, wv->ptr, kvd, H, xb->ptr, n));
    }
    // The q/k norms, the rotations and the appends (model.rs:111-120), one
    // wave per (token, head), into the trait's position-major caches.
    th::QkvPostArgs a{};
    a.q = q->ptr;
    a.k = k->ptr;
    a.v = v->ptr;
    a.q_norm = q_norm ? q_norm->ptr : nullptr;
    a.k_norm = k_norm ? k_norm->ptr : nullptr;
    a.rope = rope->ptr;
    a.k_cache = k_cache->ptr;
    a.v_cache = v_cache->ptr;
    a.head_stride = (long long)head_dim;
    a.pos_stride = (long long)kvd;
    a.pos = (long long)pos;
    a.n = (int)n;
    a.n_heads = (int)n_heads;
    a.n_kv_heads = (int)n_kv_heads;
    a.head_dim = (int)head_dim;
    a.eps = eps;
    TH_HIP(th::launch_qk_norm_rope_append(dev->stream, a));
    return TH_OK;
}

int th_gate_up_silu(th_device *dev, th_buffer *gate, th_buffer *up, const th_weight *w_gate, const th_weight *w_up,
                    const th_buffer *xb) {
    TH_REQUIRE(dev && gate && up && w_gate && w_up && xb, "th_gate_up_silu: null argument");
    TH_REQUIRE(w_gate->ndim == 2 && w_up->ndim == 2 && w_gate->shape[0] == w_up->shape[0] &&
                   w_gate->shape[1] == w_up->shape[1] && w_gate->shape[1] > 0,
               "gate and up weights of one shape");
    const size_t I = w_gate->shape[0], H = w_gate->shape[1], n = xb->len / H;
    TH_REQUIRE(n > 0 && xb->len == n * H, "xb holds %zu activations, not whole rows of %zu", xb->len, H);
    TH_REQUIRE(gate->len == n * I && up->len == n * I, "gate and up hold %zu tokens of %zu", n, I);
    TH_REQUIRE(gate->ptr != xb->ptr && up->ptr != xb->ptr && gate->ptr != up->ptr, "gate, up and xb are distinct");
    if (n == 1 && th::step_gemv_supported((int)H)) {
        // Both projections and silu(gate) * up in one GEMV launch; up unused.
        TH_HIP(th::launch_step_silu(dev->stream, w_gate->ptr, w_up->ptr, (int)I, (int)H, xb->ptr, gate->ptr));
        return TH_OK;
    }
    if (n >= th::kGemmMinTokens && th::gemm_supported(I, H)) {
        TH_NOT_CAPTURING(dev, "a projection of 16 or more tokens (stream-ordered scratch)");
        const th::GemmOut o[2] = {{w_gate->ptr, I, gate->ptr}, {w_up->ptr, I, up->ptr}};
        TH_HIP(th::launch_gemm_outs(dev->stream, xb->ptr, n, H, o, 2));
    } else {
        if (n >= th::kGemmMinTokens) TH_NOT_CAPTURING(dev, "a projection of 16 or more tokens (stream-ordered scratch)");
        TH_HIP(th::launch_matmul(dev->stream, gate->ptr, w_gate->ptr, I, H, xb->ptr, n));
        TH_HIP(th::launch_matmul(dev->stream, up->ptr, w_up->ptr, I, H, xb->ptr, n));
    }
    TH_HIP(th::launch_silu_mul(dev->stream, gate->ptr, up->ptr, n * I));
    return TH_OK;
}

int th_argmax(th_device *dev, const th_buffer *logits, uint32_t *token) {
    TH_REQUIRE(dev && logits && token, "th_argmax: null argument");
    TH_NOT_CAPTURING(dev, "th_argmax");
    TH_REQUIRE(logits->len > 0, "argmax of an empty buffer");
    size_t m = th::argmax_partials(logits->len);
    auto *partials = static_cast<uint64_t *>(th::scratch(dev, m * sizeof(uint64_t)));
    if (!partials) return fail(TH_ERR_NOMEM, "no scratch for argmax");
    TH_HIP(th::launch_argmax(dev->stream, logits->ptr, logits->len, partials, dev->token_out));
    TH_HIP(hipMemcpyAsync(token, dev->token_out, sizeof(uint32_t), hipMemcpyDeviceToHost, dev->stream));
    TH_HIP(hipStreamSynchronize(dev->stream));
    return TH_OK;
}

int th_sample(th_device *dev, const th_buffer *logits, float temperature, size_t top_k, float top_p, uint64_t *rng,
              uint32_t *token) {
    TH_REQUIRE(dev && logits && rng && token, "th_sample: null argument");
    TH_NOT_CAPTURING(dev, "th_sample");
    TH_REQUIRE(logits->len > 0, "sampling from an empty buffer");
    if (temperature == 0.0f) return th_argmax(dev, logits, token);
    const size_t k = std::min(std::max<size_t>(top_k, 1), logits->len);
    TH_REQUIRE(k <= (size_t)th::kSampleMaxTopK, "top_k %zu: the device samples from at most %d candidates", k,
               th::kSampleMaxTopK);
    TH_REQUIRE(logits->len <= th::kSampleMaxVocab, "sampling over %zu values: at most %zu", logits->len,
               th::kSampleMaxVocab);
    TH_REQUIRE(top_p > 0.0f, "top_p must be greater than 0");
    // The sampler's state, then the candidate keys.
    constexpr size_t head = 256;
    char *sc = static_cast<char *>(th::scratch(dev, head + th::sample_scratch_bytes(logits->len)));
    if (!sc) return fail(TH_ERR_NOMEM, "no scratch for sampling");
    auto *ss_dev = reinterpret_cast<th::SampleState *>(sc);
    th::SampleState ss{*rng, *rng, temperature, top_p, (int)k, 0};
    TH_HIP(hipMemcpyAsync(ss_dev, &ss, sizeof ss, hipMemcpyHostToDevice, dev->stream));
    TH_HIP(th::launch_sample(dev->stream, logits->ptr, logits->len, sc + head, ss_dev, nullptr, 0));
    TH_HIP(hipMemcpyAsync(&ss, ss_dev, sizeof ss, hipMemcpyDeviceToHost, dev->stream));
    TH_HIP(hipStreamSynchronize(dev->stream));
    *rng = ss.rng;
    *token = ss.token;
    return TH_OK;
}

}  // extern "C"
