/*
 * titania_hip_test.h: test-only entry points of the hip device library.
 *
 * Each runs one fused kernel of the decode step or of the prefill on caller
 * buffers, so that a test can hold it to the per-kernel bar (relative error
 * <= 1e-3) against the oracle's composition of the reference's primitives
 * (model/cpu.rs). They are not part of the Device boundary (titania_hip.h),
 * the forward and decode paths never call them, and they may allocate and
 * wait. Caches are f32, laid out [kv_head][max_len][128] as the fused path
 * keeps them; the rope table is [max_len][64][cos, sin] (model/model.rs:239-250).
 */
#ifndef TITANIA_HIP_TEST_H
#define TITANIA_HIP_TEST_H

#include "titania_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Decode-step q/k/v GEMV: x_out = x + y (y may be NULL), qkv = [wq; wk; wv] .
 * rmsnorm(x_out, gain) (model/model.rs:106-110 for one token). */
TH_API int th_test_step_qkv(th_device *dev, const th_weight *wq, const th_weight *wk, const th_weight *wv,
                            const th_buffer *x, const th_buffer *y, const th_weight *gain, float eps,
                            th_buffer *x_out, th_buffer *qkv_out);

/* Decode-step gate/up GEMV with the SiLU epilogue: x_out = x1 + o,
 * h = silu(gate . n) * (up . n), n = rmsnorm(x_out, gain) (model.rs:132-140). */
TH_API int th_test_step_gate_up(th_device *dev, const th_weight *gate, const th_weight *up, const th_buffer *x1,
                                const th_buffer *o, const th_weight *gain, float eps, th_buffer *x_out,
                                th_buffer *h);

/* Decode-step plain GEMV (the o and down projections): out = w . x. */
TH_API int th_test_step_gemv(th_device *dev, const th_weight *w, const th_buffer *x, th_buffer *out);

/* Decode-step output projection with the argmax epilogue and the pick:
 * logits = w . rmsnorm(x + y, gain) (model.rs:144-147), *token = the greedy
 * pick of model/sampler.rs:21-33 (lowest index on ties). */
TH_API int th_test_step_logits(th_device *dev, const th_weight *w, const th_buffer *x, const th_buffer *y,
                               const th_weight *gain, float eps, th_buffer *logits, uint32_t *token);

/* The decode step's fused q/k/v + attention launch for one token at `pos`:
 * x_out = x + y, q/k/v = the GEMV of rmsnorm(x_out); q and k RMSNorm'd per
 * head (q_norm / k_norm may be NULL) and rotated, k and v appended to the
 * caches at pos, att = attention over positions 0..pos (model.rs:106-124).
 * Past the chunked launch's reach (more than 32 chunks of 64 positions a
 * head, or 512 attention blocks), the launch that runs the streaming split
 * attention instead, then the combine. The caches extend 128 rows of 128
 * floats past the last head. */
TH_API int th_test_step_qkv_attn(th_device *dev, const th_weight *wq, const th_weight *wk, const th_weight *wv,
                                 const th_buffer *x, const th_buffer *y, const th_weight *gain,
                                 const th_weight *q_norm, const th_weight *k_norm, float eps, const th_buffer *rope,
                                 th_buffer *k_cache, th_buffer *v_cache, size_t max_len, size_t pos,
                                 size_t n_heads, size_t n_kv_heads, th_buffer *x_out, th_buffer *att_out);

/* The decode step's split attention and its combine for one token at `pos`
 * (model.rs:111-124), the launches a step takes at any context for groups of
 * 1 or 8 q heads (groups of 2 and 4 run the same attention inside the q/k/v
 * launch once the chunked launch no longer reaches): qkv holds the raw q, k and v rows
 * ([n_heads * 128][n_kv_heads * 128][n_kv_heads * 128]); q and k are
 * RMSNorm'd per head (q_norm / k_norm may be NULL) and rotated, k and v
 * appended to the caches at pos, and att = attention over positions
 * 0..pos, in the splits the step uses for caches of max_len positions,
 * merged by the combine kernel when there are several (*n_splits, if not
 * NULL, receives their count). kv_bf16 = 1: the caches hold bf16 values, two
 * to a float of the buffer. The caches extend 128 rows of 128 floats past
 * the last head. */
TH_API int th_test_step_attention(th_device *dev, const th_buffer *qkv, const th_weight *q_norm,
                                  const th_weight *k_norm, float eps, const th_buffer *rope, th_buffer *k_cache,
                                  th_buffer *v_cache, size_t max_len, size_t pos, size_t n_heads, size_t n_kv_heads,
                                  int kv_bf16, th_buffer *att_out, int *n_splits);

/* Prefill q/k/v GEMM on the matrix cores with the q/k norm + RoPE + KV
 * append epilogue, for n tokens at pos .. pos + n - 1: q_out = the rotated,
 * normalized q rows; k and v go to the caches (model.rs:108-120). xn holds
 * the normalized input rows. With `planes` (or NULL), the epilogue also
 * writes the prefill attention's bf16 planes of the new keys and values into
 * it, as bf16 pairs in its floats: K hi, K lo [n_kv_heads][L][128], V^T hi,
 * V^T lo [n_kv_heads][128][L] (L = max_len rounded up to 64; each 32-key
 * slice of a V^T row holds key 4 g + i at column 8 g + i and key
 * 16 + 4 g + i at column 8 g + 4 + i, g, i < 4); other positions are left
 * as they were. */
TH_API int th_test_gemm_qkv(th_device *dev, const th_buffer *xn, const th_weight *wq, const th_weight *wk,
                            const th_weight *wv, const th_weight *q_norm, const th_weight *k_norm, float eps,
                            const th_buffer *rope, th_buffer *k_cache, th_buffer *v_cache, size_t max_len,
                            size_t pos, size_t n, size_t n_heads, size_t n_kv_heads, th_buffer *q_out,
                            th_buffer *planes);

/* Prefill gate/up GEMM with the SiLU epilogue: h = silu(xn . gate) *
 * (xn . up) for n rows (model.rs:137-140), as the f32 sum of the bf16 hi/lo
 * terms the kernel writes for the down GEMM. */
TH_API int th_test_gemm_silu(th_device *dev, const th_buffer *xn, const th_weight *gate, const th_weight *up,
                             size_t n, th_buffer *h_out);

/* Prefill residual add of split-K partials + RMSNorm: x += parts[0] + ... +
 * parts[n_parts - 1] (each x's length), xn = rmsnorm(x, gain) as the f32 sum
 * of the bf16 hi/lo terms the kernel writes (model.rs:132-136). */
TH_API int th_test_add_rmsnorm_parts(th_device *dev, th_buffer *x, const th_buffer *parts, size_t n_parts,
                                     const th_weight *gain, float eps, th_buffer *xn);

/* Prefill attention (model.rs:121-124 for n tokens at pos .. pos + n - 1)
 * over f32 caches of max_len positions, the q rows already normalized and
 * rotated: planes = 0 runs the kernel that splits keys and values into bf16
 * hi/lo in every block, planes = 1 the one that reads them from planes split
 * once. out = [n][n_heads * 128] f32. */
TH_API int th_test_attention_prefill(th_device *dev, const th_buffer *q, const th_buffer *k_cache,
                                     const th_buffer *v_cache, size_t max_len, size_t pos, size_t n, size_t n_heads,
                                     size_t n_kv_heads, int planes, th_buffer *out);

#ifdef __cplusplus
}
#endif

#endif /* TITANIA_HIP_TEST_H */
