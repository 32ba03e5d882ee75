/*
 * Seeded synthetic weights for Qwen3-shaped models: N(0, std) rounded to bf16
 * (round to nearest even), each element a pure function of (key, index) so that
 * any tensor can be generated alone, in parallel, identically on every host.
 *
 * key = splitmix64(seed) ^ fnv1a64(tensor name); element pairs (2j, 2j+1) come
 * from one Box-Muller transform of the 64-bit hash splitmix64(key + j).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

static inline uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

static inline uint16_t to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

EXPORT uint64_t synth_key(uint64_t seed, const char *name) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (const unsigned char *p = (const unsigned char *)name; *p; ++p) {
        h ^= *p;
        h *= 0x100000001b3ull;
    }
    return splitmix64(seed) ^ h;
}

EXPORT void synth_normal_bf16(uint16_t *out, uint64_t n, uint64_t key, float std) {
    const double two_pi = 6.283185307179586476925286766559;
    long long pairs = (long long)((n + 1) / 2);
#pragma omp parallel for schedule(static)
    for (long long j = 0; j < pairs; ++j) {
        uint64_t r = splitmix64(key + (uint64_t)j);
        double u1 = ((double)(r >> 40) + 1.0) * (1.0 / 16777216.0); /* (0, 1] */
        double u2 = (double)(r & 0xffffffull) * (1.0 / 16777216.0);  /* [0, 1) */
        double rad = sqrt(-2.0 * log(u1));
        double z0 = rad * cos(two_pi * u2), z1 = rad * sin(two_pi * u2);
        uint64_t i = (uint64_t)j * 2;
        out[i] = to_bf16((float)(z0 * std));
        if (i + 1 < n) out[i + 1] = to_bf16((float)(z1 * std));
    }
}

/* Uniform token ids in [0, vocab): the i-th is splitmix64(key + i) mod vocab. */
EXPORT void synth_tokens(uint32_t *out, uint64_t n, uint64_t key, uint32_t vocab) {
    for (uint64_t i = 0; i < n; ++i) out[i] = (uint32_t)(splitmix64(key + i) % vocab);
}
