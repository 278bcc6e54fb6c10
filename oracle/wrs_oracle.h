/*
 * CPU oracle for the whisper.rs attention path -- TEST INFRASTRUCTURE ONLY.
 *
 * This is a C restatement of the reference CPU algorithm, used by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg as the parity reference and
 * as the timed CPU baseline. It is never linked into, loaded by or called from
 * the product library (whisper.rs_amd/), which must fail loudly when its HIP
 * build is missing instead of falling back to this code.
 *
 * Every entry point returns 0 on success and a negative code when the
 * reference would panic on its shape assertions, so the Python side can raise
 * the equivalent of the Rust panic.
 *
 * Parity status of each function (what pins it) is listed in the header
 * comment of wrs_oracle.c.
 */
#ifndef WRS_ORACLE_H
#define WRS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WRS_ORACLE_Q_TILE 128  /* crates/tensor/src/ops/attention.rs:13 */
#define WRS_ORACLE_KV_TILE 128 /* crates/tensor/src/ops/attention.rs:26 */

/* crates/tensor/src/ops/softmax.rs:1-23 */
void wrs_oracle_softmax_inplace(float *x, size_t n);

/* crates/tensor/src/simd.rs:4-21 (AVX2+FMA body :49-106, scalar :24-45) */
float wrs_oracle_dot_f32(const float *a, const float *b, size_t n);

/* crates/tensor/src/ops/attention.rs:68-243. n_threads<=0 uses all cores. */
int wrs_oracle_flash_attention_2(const float *q, const float *k, const float *v,
                                 size_t t_q, size_t t_kv, size_t n_heads,
                                 size_t d_model, int causal, float *out,
                                 int n_threads);

/* crates/tensor/src/ops/attention.rs:29-41 (forwards to flash_attention_2) */
int wrs_oracle_multi_head_attention(const float *q, const float *k,
                                    const float *v, size_t t_q, size_t t_kv,
                                    size_t n_heads, size_t d_model, int causal,
                                    float *out, int n_threads);

/* crates/tensor/src/ops/attention.rs:246-434 (one query per head, d_head 64) */
/* bench_flash_attention_tiled.rs:46-107: the materialized (full score
 * matrix per head) attention the reference benchmarks the tiled kernel
 * against. */
int wrs_oracle_materialized_attention(const float *q, const float *k, const float *v,
                                      size_t t_q, size_t t_kv, size_t n_heads,
                                      size_t d_model, float *out, int n_threads);
int wrs_oracle_single_token_mha_d64(const float *q, const float *k,
                                    const float *v, size_t t_kv,
                                    size_t n_heads, size_t d_model, float *out);

/* crates/whisper/src/decoder.rs:835-892 (causal attention with offset t_past) */
int wrs_oracle_mha_with_cache(const float *q, const float *k, const float *v,
                              size_t n_tokens, size_t total_tokens,
                              size_t t_past, size_t n_heads, size_t d_model,
                              float *out);

/* decoder.rs:796-828: softmax cross-attention weights of selected heads,
 * out[((row_offset + i) * n_selected + slots[p]) * n_audio + j]. */
int wrs_oracle_capture_cross_heads(const float *q, const float *k, size_t n_tokens,
                                   size_t n_audio, size_t n_heads, size_t d_model,
                                   const size_t *slots, const size_t *heads, size_t n_pairs,
                                   size_t n_selected, size_t row_offset, float *out);

/* simd.rs:593-700 dot_f16_f32 (f16 weights widened exactly, f32 x). */
float wrs_oracle_dot_f16_f32(const uint16_t *w, const float *x, size_t len);
float wrs_oracle_f16_to_f32(uint16_t h);
/* quant.rs:415-473 f16_linear: out[t * rows + r] = W[r] . x[t] + bias[r]
 * (bias may be NULL). n_threads <= 0 uses every core. */
int wrs_oracle_f16_linear(const uint16_t *w, size_t rows, size_t cols, const float *x,
                          const float *bias, size_t num_tokens, float *out, int n_threads);

/* norm.rs:116-143 layer_norm (rows of d_model, gamma/beta of d_model). */
int wrs_oracle_layer_norm(const float *in, const float *gamma, const float *beta, float eps,
                          size_t num_tokens, size_t d_model, float *out);
/* gelu.rs:3-23 (tanh form). */
float wrs_oracle_gelu(float x);
void wrs_oracle_gelu_inplace(float *data, size_t n);

/* xorshift32 generator of crates/tensor/tests/test_flash_attention_tiled.rs:15-35.
 * Fills out[0..n) and advances *state. */
void wrs_oracle_xorshift_fill(uint32_t *state, float *out, size_t n);

/* 1 when the AVX2+FMA bodies are in use (the reference's runtime dispatch,
 * crates/tensor/src/ops/attention.rs:259-269), 0 for the scalar bodies. */
int wrs_oracle_uses_avx2(void);
/* Force the scalar bodies (1) or restore runtime dispatch (0); for tests. */
void wrs_oracle_force_scalar(int on);

#ifdef __cplusplus
}
#endif
#endif
