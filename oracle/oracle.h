/*
 * oracle.h - CPU restatement of aot-llm's quantized inference path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker and the CPU
 * baseline. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it. The product (aot-llm_amd/) never links, loads or calls
 * anything here.
 *
 * The reference (p10node/aot-llm) is Rust and cannot be built in this image
 * (no cargo/rustc), so every function below restates the reference's
 * algorithm from its source, citing file:line (paths relative to the
 * reference's repository root). The x86 kernel set restated is `avx2+f16c`
 * (crates/aot-kernels/src/matvec.rs:248-253), with the same intrinsics in
 * the same order, so its float results are reproduced bit for bit. Built with
 * -ffp-contract=off (Rust never contracts a*b+c into an FMA outside explicit
 * intrinsics).
 *
 * Parity pinning (what checks each part, see tests/test_oracle.py):
 *   f16/bf16 converters      known values quant.rs:456-463 + exhaustive
 *                            round trip of all 65536 halves
 *   quantize_q8_0 / q8_k     reconstruction bound quant.rs:466-479, bsums
 *                            invariant quant.rs:481-490, closed-form scale
 *   encoders quantize_row_*  round-trip error bounds quantize.rs:322-333 and
 *                            re-encoding of exactly representable rows
 *   dequant_row_*            brute-force bit unpacking of random blocks
 *   dots (scalar, avx2, x4)  f64 dequantized reference (tests/dots.rs:52-89),
 *                            exact-integer recomputation, x4 == single
 *                            (dots.rs:161-203), matmul == matvec
 *                            (dots.rs:207-266), parallel == serial
 *   ops                      closed forms of ops.rs:220-351
 *   forward / forward_batch  batched == token-by-token bitwise (README.md:183)
 *                            and an f64 activation-quantizing reference
 *                            forward (e2e.rs:160-343) within its tolerance
 * Parity unpinned (no Rust run possible): the ulp-level results of glibc's
 * expf/tanhf/sinf/cosf/powf as called from Rust (assumed identical, both
 * call glibc on Linux) and the exact avx2 float order of the Q8_0-family and
 * float dots (deterministic from the intrinsic sequence, restated, pinned to
 * the reference's own 1e-4 scalar tolerance).
 */
#ifndef AOTK_ORACLE_H
#define AOTK_ORACLE_H

#include <stddef.h>
#include <stdint.h>
#include "../include/aotk.h"

#ifdef __cplusplus
extern "C" {
#endif

/* quant.rs:96-177 */
float or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);
float or_bf16_to_f32(uint16_t h);
uint16_t or_f32_to_bf16(float f);

size_t or_row_bytes(int kind, size_t cols);

/* quant.rs:231-283 */
void or_quantize_q8_0(const float *x, size_t n, aotk_block_q8_0 *out);
void or_quantize_q8_k(const float *x, size_t n, aotk_block_q8_k *out);

/* quant.rs:300-443 */
void or_dequant_row(int kind, const uint8_t *row, float *out, size_t n);
/* quantize.rs:282-294; returns bytes written */
size_t or_quantize_row(int kind, const float *x, size_t n, uint8_t *out);

/* matvec.rs:30-192 (scalar) and simd_avx2.rs (avx2). x is aotk_block_q8_0*,
 * aotk_block_q8_k* or float* depending on kind. */
float or_dot_scalar(int kind, const uint8_t *w, const void *x, size_t cols);
float or_dot_avx2(int kind, const uint8_t *w, const void *x, size_t cols);
/* 1x4 micro-kernels (simd_avx2.rs:273-430); returns -1 when the kind has
 * none (Q5_K, floats: matvec.rs:537-546). */
int or_dot_avx2_x4(int kind, const uint8_t *w, const void *const xs[4], size_t cols, float out[4]);

/* fork-join pool (pool.rs) */
typedef struct or_pool or_pool;
or_pool *or_pool_new(int n_threads);
void or_pool_free(or_pool *p);
int or_pool_threads(const or_pool *p);

/* matvec.rs:300-401 and :468-546; kernels: 0 = scalar, 1 = avx2+f16c */
void or_matvec(or_pool *p, int kernels, int kind, float *out, const uint8_t *w, const void *x, size_t rows, size_t cols);
void or_matmul(or_pool *p, int kernels, int kind, float *out, const uint8_t *w, const void *xs, size_t m, size_t rows, size_t cols);

/* ops.rs */
void or_rmsnorm(float *out, const float *x, const float *w, size_t n, float eps);
void or_rope_cos_sin(float *cs, const float *inv_freq, size_t half, float pos);
void or_rope(float *x, size_t n_heads, size_t head_dim, size_t rot_dim, const float *cs, int neox);
void or_rmsnorm_heads(float *x, const float *w, size_t n_heads, size_t head_dim, float eps);
void or_softmax(float *x, size_t n);
void or_silu_mul(float *h, const float *up, size_t n);
float or_gelu(float v);
void or_gelu_mul(float *h, const float *up, size_t n);
size_t or_window_start(size_t pos, size_t window);
void or_attention(or_pool *p, float *out, const float *q, const float *k_cache, const float *v_cache,
                  size_t n_head, size_t n_kv_head, size_t head_dim, size_t ctx, size_t layer,
                  size_t pos0, size_t m, size_t window);
void or_inv_freq(float *out, size_t rot_dim, float base, const float *factors);
uint32_t or_argmax(const float *x, size_t n);
/* sampler.rs: splitmix seeding (:113-118) and Sampler::sample (:47-96) with
 * the rng state in *rng; ties of equal scaled logits in ascending id order. */
uint64_t or_sampler_seed(uint64_t seed);
uint32_t or_sample(const aotk_sampler_config *cfg, uint64_t *rng, float *logits, size_t n, const uint32_t *recent,
                   size_t n_recent);

/* Synthetic weights: tests and the bench build their models from this
 * generator (shared definition with the product's device generator). */
float or_synth_value(uint64_t seed, uint32_t tensor_index, uint64_t elem);
/* Fill the blob for spec with encoded synthetic tensors. Tensor index of a
 * spec slot: token_embd 0, output_norm 1, output 2, layer l slot s (in
 * aotk_layer field order) 3 + 16*l + s. */
int or_synth_blob(const aotk_model_spec *spec, uint64_t seed, uint8_t *blob, size_t blob_len, int n_threads);

/* crates/aot-llm/tests/e2e.rs:81-95 `Rng`: xorshift64 (13, 7, 17) with
 * uniform(a) = ((next % 1000001) as f32 / 500000 - 1) * a; fills out[0..n)
 * in stream order and advances *state. */
void or_e2e_uniform(uint64_t *state, float a, float *out, size_t n);

/* Model runtime (state.rs, emit.rs forward/forward_batch) */
typedef struct or_model or_model;
or_model *or_model_new(const aotk_model_spec *spec, const uint8_t *blob, size_t blob_len,
                       size_t ctx, size_t max_batch, int n_threads, int kernels);
void or_model_free(or_model *m);
int or_forward(or_model *m, uint32_t token, size_t pos, int want_logits);
int or_forward_batch(or_model *m, const uint32_t *tokens, size_t n, size_t pos0, int want_logits);
const float *or_logits(const or_model *m);
float *or_k_cache(or_model *m);
float *or_v_cache(or_model *m);

#ifdef __cplusplus
}
#endif
#endif
