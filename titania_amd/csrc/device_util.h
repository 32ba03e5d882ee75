// Device-side helpers shared by the kernels: bf16 unpacking, wave64
// reductions, the SiLU activation and the packed argmax key.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace th {

// bf16 is the top half of an f32 (model/cpu.rs:158-161).
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Eight bf16 (one 16-byte load) to f32, element order preserved.
__device__ __forceinline__ void unpack8(const uint4 &w, float f[8]) {
    f[0] = bf16_lo(w.x); f[1] = bf16_hi(w.x);
    f[2] = bf16_lo(w.y); f[3] = bf16_hi(w.y);
    f[4] = bf16_lo(w.z); f[5] = bf16_hi(w.z);
    f[6] = bf16_lo(w.w); f[7] = bf16_hi(w.w);
}

// 16-byte loads with the non-temporal (streaming) cache policy, for weight
// rows that a decode step reads once. On the Qwen3-0.6B decode step this took
// 0.605 to 0.570 ms against plain loads (the same policy on the cached key
// and value rows made the step slower; the scope bits sc0 / sc1 changed
// nothing beside it).
typedef unsigned int th_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_nt(const uint4 *p) {
    const th_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const th_u32x4 *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
// The same through a buffer descriptor of a wave-uniform row base (the
// address lives in scalar registers: 0.570 -> 0.567 ms on that step).
// Element idx of the row, idx * 16 < 2^31.
constexpr int kCachePolicyNt = 2;               // the instruction's nt bit
constexpr unsigned kBufferRsrcWord3 = 0x00020000;  // raw 32-bit data, no swizzle
__device__ __forceinline__ uint4 ld_nt_row(const uint4 *row, int idx) {
    __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint4 *>(row), 0, 0x7fffffff,
                                                                 kBufferRsrcWord3);
    const th_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, idx * 16, 0, kCachePolicyNt);
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Round-to-nearest-even f32 -> bf16 bits (finite inputs; NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// An f32 as two bf16 terms, x ~ hi + lo with hi = bf16(x), lo = bf16(x - hi)
// (round to nearest even, the hardware conversion): 16 significant bits
// together. The matrix-core GEMM takes its activations in this form.
typedef __bf16 th_bf16x2 __attribute__((ext_vector_type(2)));
typedef float th_f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void split_bf16(float x, uint16_t &hi, uint16_t &lo) {
    const __bf16 h = (__bf16)x;
    hi = __builtin_bit_cast(uint16_t, h);
    lo = __builtin_bit_cast(uint16_t, (__bf16)(x - (float)h));
}

__device__ __forceinline__ void split_bf16x4(const float4 &v, uint2 &hi, uint2 &lo) {
    const th_bf16x2 h01 = __builtin_convertvector((th_f32x2){v.x, v.y}, th_bf16x2);
    const th_bf16x2 h23 = __builtin_convertvector((th_f32x2){v.z, v.w}, th_bf16x2);
    const uint32_t u01 = __builtin_bit_cast(uint32_t, h01), u23 = __builtin_bit_cast(uint32_t, h23);
    const th_bf16x2 l01 = __builtin_convertvector(
        (th_f32x2){v.x - __uint_as_float(u01 << 16), v.y - __uint_as_float(u01 & 0xffff0000u)}, th_bf16x2);
    const th_bf16x2 l23 = __builtin_convertvector(
        (th_f32x2){v.z - __uint_as_float(u23 << 16), v.w - __uint_as_float(u23 & 0xffff0000u)}, th_bf16x2);
    hi = make_uint2(u01, u23);
    lo = make_uint2(__builtin_bit_cast(uint32_t, l01), __builtin_bit_cast(uint32_t, l23));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Wave64 sum through DPP: butterfly within each 16-lane row, then row
// broadcasts; the total ends in lane 63 and is read back as a scalar.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float v) {
    const int t = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false);
    return v + __int_as_float(t);
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
    v = dpp_add<0xB1, 0xf>(v);   // quad_perm [1,0,3,2]
    v = dpp_add<0x4E, 0xf>(v);   // quad_perm [2,3,0,1]
    v = dpp_add<0x124, 0xf>(v);  // row_ror:4
    v = dpp_add<0x128, 0xf>(v);  // row_ror:8
    v = dpp_add<0x142, 0xa>(v);  // row_bcast:15
    v = dpp_add<0x143, 0xc>(v);  // row_bcast:31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// v from another lane of the same 16-lane row (or across rows for the
// row_bcast controls); lanes whose row is not in ROW_MASK get `old`.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_get(float v, float old) {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

// Sum over each 16-lane row, left in every lane of the row (the association
// differs between lanes, so callers use one lane's value).
__device__ __forceinline__ float row_sum_dpp(float v) {
    v += dpp_get<0xB1>(v, 0.f);   // quad_perm [1,0,3,2]
    v += dpp_get<0x4E>(v, 0.f);   // quad_perm [2,3,0,1]
    v += dpp_get<0x124>(v, 0.f);  // row_ror:4
    v += dpp_get<0x128>(v, 0.f);  // row_ror:8
    return v;
}

// Wave64 maximum through DPP, returned to every lane.
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp_get<0xB1>(v, -INFINITY));
    v = fmaxf(v, dpp_get<0x4E>(v, -INFINITY));
    v = fmaxf(v, dpp_get<0x124>(v, -INFINITY));
    v = fmaxf(v, dpp_get<0x128>(v, -INFINITY));
    v = fmaxf(v, dpp_get<0x142, 0xa>(v, -INFINITY));  // row_bcast:15
    v = fmaxf(v, dpp_get<0x143, 0xc>(v, -INFINITY));  // row_bcast:31
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// The maximum (sum) of v over lanes l, l ^ 16 and l ^ 32, l ^ 48: the four
// 16-lane rows of a wave combined lane by lane, in every lane. gfx950's
// permlane swaps exchange whole rows in the VALU (no LDS round trip); since
// max and + commute, every lane gets the same (r0 op r1) op (r2 op r3).
__device__ __forceinline__ float rows_max(float v) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
// rows_max for values that are never NaN: a plain v_max_f32 (fmaxf brings
// a NaN canonicalization of each input with it).
__device__ __forceinline__ float max_nn(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ float rows_max_nn(float v) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = max_nn(__uint_as_float(p[0]), __uint_as_float(p[1]));
    auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return max_nn(__uint_as_float(q[0]), __uint_as_float(q[1]));
}
__device__ __forceinline__ float rows_sum(float v) {
    auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// Sum over aligned groups of `width` lanes (width a power of two <= 64).
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        uint64_t other = __shfl_xor(v, o, 64);
        v = max_u64(v, other);
    }
    return v;
}

// f32 under IEEE total order (Rust's f32::total_cmp) as an unsigned key, packed
// above the inverted index so that the u64 maximum is the largest value at the
// lowest index.
__device__ __forceinline__ uint64_t argmax_pack(float f, uint32_t idx) {
    int32_t k = __float_as_int(f);
    k ^= (int32_t)(((uint32_t)(k >> 31)) >> 1);
    uint32_t key = (uint32_t)k ^ 0x80000000u;
    return ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - idx);
}

__device__ __forceinline__ uint32_t argmax_index(uint64_t packed) {
    return 0xffffffffu - (uint32_t)(packed & 0xffffffffu);
}

// One 16-byte direct global -> LDS load a lane (global_load_lds): lane l's
// 16 bytes land at lds_wave_base + 16 l, so a wave fills one 1 KB span; the
// LDS address must be the same in every lane of the wave.
__device__ __forceinline__ void dma16(const void *src, uint4 *lds_wave_base) {
    __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void *)lds_wave_base, 16, 0, 0);
}

// s_waitcnt vmcnt(N) leaving the other counters alone (gfx9 encoding): a
// global_load_lds counts until its LDS write is done.
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

// model/cpu.rs:153: g / (1 + exp(-g)).
__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

}  // namespace th
