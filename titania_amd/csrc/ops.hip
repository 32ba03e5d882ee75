// Elementwise and row-wise kernels of the Device operations: embed, copy, add,
// silu_mul, rmsnorm (with an optional fused residual add), rope and argmax.
// All are HBM- or latency-bound; each works on f32 activations with bf16 gains.
#include "common.h"
#include "device_util.h"

namespace th {

// model/cpu.rs:38-47: out[t][i] = bf16(table[tokens[t]][i]). One block per token;
// 8 bf16 per 16-byte load when dim allows.
__global__ void embed_kernel(float *__restrict__ out, const uint16_t *__restrict__ table, size_t dim,
                             const uint32_t *__restrict__ tokens) {
    const size_t t = blockIdx.x;
    const uint16_t *row = table + (size_t)tokens[t] * dim;
    float *o = out + t * dim;
    if ((dim & 7) == 0) {
        for (size_t c = threadIdx.x; c < dim / 8; c += blockDim.x) {
            uint4 w = *reinterpret_cast<const uint4 *>(row + c * 8);
            float f[8];
            unpack8(w, f);
            float4 *o4 = reinterpret_cast<float4 *>(o + c * 8);
            o4[0] = make_float4(f[0], f[1], f[2], f[3]);
            o4[1] = make_float4(f[4], f[5], f[6], f[7]);
        }
    } else {
        for (size_t i = threadIdx.x; i < dim; i += blockDim.x) o[i] = bf16_to_f32(row[i]);
    }
}

hipError_t launch_embed(hipStream_t s, float *out, const uint16_t *table, size_t dim, const uint32_t *tokens,
                        size_t n) {
    if (n == 0) return hipSuccess;
    embed_kernel<<<dim3((unsigned)n), dim3(256), 0, s>>>(out, table, dim, tokens);
    return hipGetLastError();
}

__global__ void copy_kernel(float *__restrict__ dst, const float *__restrict__ src, size_t len) {
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len; i += stride) dst[i] = src[i];
}

// Overlapping ranges (model/device.rs:34-42 allows dst and src to be the same
// buffer) are copied through a memmove on the stream instead.
hipError_t launch_copy(hipStream_t s, float *dst, const float *src, size_t len) {
    if (len == 0 || dst == src) return hipSuccess;
    bool overlap = (dst < src + len) && (src < dst + len);
    if (overlap) return hipMemcpyAsync(dst, src, len * sizeof(float), hipMemcpyDeviceToDevice, s);
    unsigned blocks = (unsigned)std::min<size_t>((len + 255) / 256, 4096);
    copy_kernel<<<blocks, 256, 0, s>>>(dst, src, len);
    return hipGetLastError();
}

__global__ void add_kernel(float *__restrict__ x, const float *__restrict__ y, size_t len) {
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len; i += stride) x[i] = x[i] + y[i];
}

hipError_t launch_add(hipStream_t s, float *x, const float *y, size_t len) {
    if (len == 0) return hipSuccess;
    unsigned blocks = (unsigned)std::min<size_t>((len + 255) / 256, 4096);
    add_kernel<<<blocks, 256, 0, s>>>(x, y, len);
    return hipGetLastError();
}

// model/cpu.rs:151-155: g = g / (1 + exp(-g)) * u.
__global__ void silu_mul_kernel(float *__restrict__ g, const float *__restrict__ u, size_t len) {
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len; i += stride) g[i] = silu(g[i]) * u[i];
}

hipError_t launch_silu_mul(hipStream_t s, float *gate, const float *up, size_t len) {
    if (len == 0) return hipSuccess;
    unsigned blocks = (unsigned)std::min<size_t>((len + 255) / 256, 4096);
    silu_mul_kernel<<<blocks, 256, 0, s>>>(gate, up, len);
    return hipGetLastError();
}

// The same product as split_bf16 terms (the down projection's GEMM input), 4
// elements a thread.
__global__ void silu_mul_split_kernel(const float4 *__restrict__ g, const float4 *__restrict__ u,
                                      uint2 *__restrict__ hi, uint2 *__restrict__ lo, size_t len4) {
    size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < len4; i += stride) {
        const float4 a = g[i], b = u[i];
        split_bf16x4(make_float4(silu(a.x) * b.x, silu(a.y) * b.y, silu(a.z) * b.z, silu(a.w) * b.w), hi[i], lo[i]);
    }
}

hipError_t launch_silu_mul_split(hipStream_t s, const float *gate, const float *up, size_t len, uint16_t *hi,
                                 uint16_t *lo) {
    if (len == 0) return hipSuccess;
    if (len % 4 || ((uintptr_t)gate | (uintptr_t)up) % 16 || ((uintptr_t)hi | (uintptr_t)lo) % 8)
        return hipErrorInvalidValue;
    const size_t len4 = len / 4;
    unsigned blocks = (unsigned)std::min<size_t>((len4 + 255) / 256, 4096);
    silu_mul_split_kernel<<<blocks, 256, 0, s>>>(reinterpret_cast<const float4 *>(gate),
                                                 reinterpret_cast<const float4 *>(up), reinterpret_cast<uint2 *>(hi),
                                                 reinterpret_cast<uint2 *>(lo), len4);
    return hipGetLastError();
}

// model/cpu.rs:85-94, optionally preceded by the residual add of
// model/model.rs:132/141: one wave per dim-long row. The residual, if any, is
// the sum of ny partial products y[z * y_stride] taken in z order (a GEMM's
// split-K partials, or ny = 1 for a plain vector); x += residual is stored
// back into x. The normalized row goes to xb (f32, which may be x) and/or, as
// split_bf16 terms, to hi/lo for the next matrix-core GEMM.
// NV > 0: dim == 256 * NV, each lane holds NV float4 of the row and issues all
// their loads before using any (one memory round trip per row); NV == 0: any
// dim, element by element.
struct NormArgs {
    float *x;
    const float *y;
    int ny;
    size_t y_stride;
    float *xb;
    uint16_t *hi, *lo;
    size_t rows;
    const uint16_t *w;
    size_t dim;
    float eps;
};

template <int NV>
// The fields the first loads need lead the parameters (preloaded into
// SGPRs); the rest of a is read as the epilogue needs it.
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(float *__restrict__ ax, const float *__restrict__ ay,
                                                          const uint16_t *__restrict__ aw, size_t arows, size_t adim,
                                                          size_t ay_stride, int any, NormArgs a) {
    const size_t row = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= arows) return;
    const size_t dim = adim;
    float *xr = ax + row * dim;
    const float *yr = any ? ay + row * dim : nullptr;
    float ss = 0.f;
    if (NV > 0) {
        float4 v[NV > 0 ? NV : 1], u[NV > 0 ? NV : 1];
        uint2 g[NV > 0 ? NV : 1];
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const int i = lane + 64 * k;
            v[k] = reinterpret_cast<const float4 *>(xr)[i];
            if (yr) u[k] = reinterpret_cast<const float4 *>(yr)[i];
            g[k] = reinterpret_cast<const uint2 *>(aw)[i];
        }
        for (int z = 1; z < any; ++z) {
            const float4 *yz = reinterpret_cast<const float4 *>(yr + (size_t)z * ay_stride);
            float4 t[NV > 0 ? NV : 1];
#pragma unroll
            for (int k = 0; k < NV; ++k) t[k] = yz[lane + 64 * k];
#pragma unroll
            for (int k = 0; k < NV; ++k) {
                u[k].x += t[k].x;
                u[k].y += t[k].y;
                u[k].z += t[k].z;
                u[k].w += t[k].w;
            }
        }
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            if (yr) {
                v[k].x = v[k].x + u[k].x;
                v[k].y = v[k].y + u[k].y;
                v[k].z = v[k].z + u[k].z;
                v[k].w = v[k].w + u[k].w;
                reinterpret_cast<float4 *>(xr)[lane + 64 * k] = v[k];
            }
            ss += v[k].x * v[k].x + v[k].y * v[k].y + v[k].z * v[k].z + v[k].w * v[k].w;
        }
        const float scale = 1.0f / sqrtf(wave_sum_dpp(ss) / (float)dim + a.eps);
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            float4 o;
            o.x = v[k].x * (scale * bf16_lo(g[k].x));
            o.y = v[k].y * (scale * bf16_hi(g[k].x));
            o.z = v[k].z * (scale * bf16_lo(g[k].y));
            o.w = v[k].w * (scale * bf16_hi(g[k].y));
            const size_t i = row * dim / 4 + lane + 64 * k;
            if (a.xb) reinterpret_cast<float4 *>(a.xb)[i] = o;
            if (a.hi) split_bf16x4(o, reinterpret_cast<uint2 *>(a.hi)[i], reinterpret_cast<uint2 *>(a.lo)[i]);
        }
        return;
    }
    for (size_t i = lane; i < dim; i += 64) {
        float v = xr[i];
        if (yr) {
            float u = yr[i];
            for (int z = 1; z < any; ++z) u += yr[(size_t)z * ay_stride + i];
            v = v + u;
            xr[i] = v;
        }
        ss += v * v;
    }
    ss = wave_sum(ss);
    const float scale = 1.0f / sqrtf(ss / (float)dim + a.eps);
    for (size_t i = lane; i < dim; i += 64) {
        const float o = xr[i] * (scale * bf16_to_f32(aw[i]));
        if (a.xb) a.xb[row * dim + i] = o;
        if (a.hi) split_bf16(o, a.hi[row * dim + i], a.lo[row * dim + i]);
    }
}

hipError_t launch_add_rmsnorm_parts(hipStream_t s, float *x, const float *y, int ny, size_t y_stride, float *xb,
                                    uint16_t *hi, uint16_t *lo, size_t rows, const uint16_t *w, size_t dim,
                                    float eps) {
    if (rows == 0) return hipSuccess;
    if (ny < 0 || (ny > 0 && !y) || (!xb && !hi) || (!hi != !lo)) return hipErrorInvalidValue;
    const NormArgs a{x, ny ? y : nullptr, ny, y_stride, xb, hi, lo, rows, w, dim, eps};
    const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
    // Row views as float4 (and hi/lo as uint2) need 16-byte (8-byte) alignment;
    // the device's buffers have it.
    const bool vec = dim % 256 == 0 && y_stride % 4 == 0 &&
                     ((uintptr_t)x | (uintptr_t)xb | (uintptr_t)a.y | (uintptr_t)w) % 16 == 0 &&
                     ((uintptr_t)hi | (uintptr_t)lo) % 8 == 0;
    switch (vec ? dim / 256 : 0) {
    case 1: add_rmsnorm_kernel<1><<<grid, block, 0, s>>>(a.x, a.y, a.w, a.rows, a.dim, a.y_stride, a.ny, a); break;
    case 2: add_rmsnorm_kernel<2><<<grid, block, 0, s>>>(a.x, a.y, a.w, a.rows, a.dim, a.y_stride, a.ny, a); break;
    case 4: add_rmsnorm_kernel<4><<<grid, block, 0, s>>>(a.x, a.y, a.w, a.rows, a.dim, a.y_stride, a.ny, a); break;
    case 8: add_rmsnorm_kernel<8><<<grid, block, 0, s>>>(a.x, a.y, a.w, a.rows, a.dim, a.y_stride, a.ny, a); break;
    case 10: add_rmsnorm_kernel<10><<<grid, block, 0, s>>>(a.x, a.y, a.w, a.rows, a.dim, a.y_stride, a.ny, a); break;
    case 16: add_rmsnorm_kernel<16><<<grid, block, 0, s>>>(a.x, a.y, a.w, a.rows, a.dim, a.y_stride, a.ny, a); break;
    default: add_rmsnorm_kernel<0><<<grid, block, 0, s>>>(a.x, a.y, a.w, a.rows, a.dim, a.y_stride, a.ny, a); break;
    }
    return hipGetLastError();
}

hipError_t launch_add_rmsnorm(hipStream_t s, float *x, const float *y, float *xb, size_t rows, const uint16_t *w,
                              size_t dim, float eps) {
    return launch_add_rmsnorm_parts(s, x, y, y ? 1 : 0, 0, xb, nullptr, nullptr, rows, w, dim, eps);
}

hipError_t launch_rmsnorm(hipStream_t s, float *x, size_t rows, const uint16_t *w, size_t dim, float eps) {
    return launch_add_rmsnorm(s, x, nullptr, x, rows, w, dim, eps);
}

// model/cpu.rs:96-111: one block per (token, head), one thread per pair.
__global__ void rope_kernel(float *__restrict__ x, const float *__restrict__ table, size_t pos, size_t n_heads,
                            size_t head_dim) {
    const size_t t = blockIdx.x / n_heads, h = blockIdx.x % n_heads;
    const size_t half = head_dim / 2;
    float *head = x + (t * n_heads + h) * head_dim;
    const float *ang = table + (pos + t) * head_dim;
    for (size_t i = threadIdx.x; i < half; i += blockDim.x) {
        float c = ang[2 * i], sn = ang[2 * i + 1];
        float a = head[i], b = head[i + half];
        head[i] = a * c - b * sn;
        head[i + half] = b * c + a * sn;
    }
}

hipError_t launch_rope(hipStream_t s, float *x, size_t n, const float *table, size_t pos, size_t n_heads,
                       size_t head_dim) {
    if (n == 0 || n_heads == 0) return hipSuccess;
    unsigned threads = (unsigned)std::min<size_t>(std::max<size_t>(head_dim / 2, 64), 256);
    rope_kernel<<<dim3((unsigned)(n * n_heads)), dim3(threads), 0, s>>>(x, table, pos, n_heads, head_dim);
    return hipGetLastError();
}

// Greedy argmax (model/sampler.rs:21-33 at temperature 0). Each block reduces
// a slice to a packed (total-order key, inverted index) u64; a second pass of
// one block reduces the partials. The max of the packed values is the largest
// logit, lowest index on ties.
constexpr size_t kArgmaxSlice = 4096;

size_t argmax_partials(size_t n) { return (n + kArgmaxSlice - 1) / kArgmaxSlice; }

__global__ __launch_bounds__(256) void argmax_partial_kernel(const float *__restrict__ x, size_t n,
                                                             uint64_t *__restrict__ partials) {
    __shared__ uint64_t red[4];
    const size_t begin = (size_t)blockIdx.x * kArgmaxSlice;
    const size_t end = begin + kArgmaxSlice < n ? begin + kArgmaxSlice : n;
    uint64_t best = 0;
    for (size_t i = begin + threadIdx.x; i < end; i += 256) best = max_u64(best, argmax_pack(x[i], (uint32_t)i));
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) partials[blockIdx.x] = max_u64(max_u64(red[0], red[1]), max_u64(red[2], red[3]));
}

__global__ __launch_bounds__(256) void argmax_final_kernel(const uint64_t *__restrict__ partials, size_t m,
                                                           uint32_t *__restrict__ token) {
    __shared__ uint64_t red[4];
    uint64_t best = 0;
    for (size_t i = threadIdx.x; i < m; i += 256) best = max_u64(best, partials[i]);
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = max_u64(max_u64(red[0], red[1]), max_u64(red[2], red[3]));
        *token = argmax_index(b);
    }
}

hipError_t launch_argmax_partials(hipStream_t s, const float *x, size_t n, uint64_t *partials) {
    argmax_partial_kernel<<<dim3((unsigned)argmax_partials(n)), dim3(256), 0, s>>>(x, n, partials);
    return hipGetLastError();
}

hipError_t launch_argmax(hipStream_t s, const float *x, size_t n, uint64_t *partials, uint32_t *token) {
    size_t m = argmax_partials(n);
    hipError_t e = launch_argmax_partials(s, x, n, partials);
    if (e != hipSuccess) return e;
    argmax_final_kernel<<<1, 256, 0, s>>>(partials, m, token);
    return hipGetLastError();
}

}  // namespace th
