/*
 * aotk.h - C ABI of the MI355X (gfx950) implementation of aot-llm's quantized
 * inference hot path.
 *
 * Everything here is plain C: pointers, sizes and POD structs, no C++ or torch
 * types. A Rust FFI crate (the reference's intended caller) binds it with
 * `extern "C"` declarations; Python binds it with ctypes (aot-llm_amd/aotk).
 *
 * Conventions (mirroring crates/aot-kernels/src/capi.rs:129-141 and
 * crates/aot-codegen/src/aot_llm.h:56-62):
 *   - every entry point returns 0 on success and -1 on failure (pointer
 *     returning calls return NULL), and the reason is available from
 *     aotk_last_error() (thread-local string);
 *   - calls are synchronous with respect to the host unless documented
 *     otherwise; all device work is issued on the library's own HIP stream;
 *   - the library is single-threaded per model/state, like the reference's
 *     `&mut Gpu` handle (crates/aot-kernels/src/metal.rs:331-520) and the
 *     `Model.lock` serialisation of aot_eval (capi.rs:181, :485).
 *
 * Pointers named *_dev are device (HBM) addresses allocated with
 * aotk_dev_alloc (or any hipMalloc'd memory of the same device).
 */
#ifndef AOTK_H
#define AOTK_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------ */
/* Formats                                                                   */
/* ------------------------------------------------------------------------ */

/* Weight element kinds: crates/aot-kernels/src/quant.rs:35-87 (`Kind`). */
enum aotk_kind {
    AOTK_F32 = 0,
    AOTK_F16 = 1,
    AOTK_BF16 = 2,
    AOTK_Q4_0 = 3,
    AOTK_Q5_0 = 4,
    AOTK_Q8_0 = 5,
    AOTK_Q4_K = 6,
    AOTK_Q5_K = 7,
    AOTK_Q6_K = 8,
    AOTK_KIND_NONE = -1
};

/* Activation blocks, byte-compatible with the reference's #[repr(C)]
 * structs: BlockQ8_0 (quant.rs:194-199, 36 bytes) and BlockQ8_K
 * (quant.rs:210-216, 292 bytes). */
typedef struct aotk_block_q8_0 {
    float d;
    int8_t qs[32];
} aotk_block_q8_0;

typedef struct aotk_block_q8_k {
    float d;
    int8_t qs[256];
    int16_t bsums[16];
} aotk_block_q8_k;

/* One tensor of the weight blob: crates/aot-kernels/src/state.rs:165-180
 * (`Tensor {kind, off, len, rows, cols}`). kind == AOTK_KIND_NONE marks an
 * absent optional tensor. Matrices are row-major, `rows` outputs x `cols`
 * inputs (ggml order), rows are `row_bytes(kind, cols)` apart. */
typedef struct aotk_tensor {
    int32_t kind;
    int32_t reserved;
    uint64_t off;
    uint64_t len;
    uint64_t rows;
    uint64_t cols;
} aotk_tensor;

/* Hyper-parameters: crates/aot-kernels/src/state.rs:126-161 (`Dims`). */
typedef struct aotk_dims {
    uint64_t dim, hidden, n_layer, n_head, n_kv_head, head_dim, rot_dim, vocab, n_ctx_train;
    float eps, rope_base, rope_scale;
    uint32_t swa_window;
    float rope_base_local, rope_scale_local;
} aotk_dims;

/* Architecture switches: crates/aot-codegen/src/model.rs:152-192
 * (`ArchFlags`; fused_qkv/fused_gate_up are row views resolved by the
 * caller into separate tensors, model.rs:352-363). */
typedef struct aotk_flags {
    uint8_t rope_neox, qkv_bias, qk_norm, embd_scale, post_norms, gelu;
    uint8_t reserved[2];
    uint32_t swa_pattern;
} aotk_flags;

/* Per-layer tensors: crates/aot-codegen/src/model.rs:121-148 (`LayerSpec`). */
typedef struct aotk_layer {
    aotk_tensor attn_norm, wq, wk, wv, wo, ffn_norm, gate, up, down;
    aotk_tensor bq, bk, bv, q_norm, k_norm, attn_post_norm, ffn_post_norm;
    int32_t local_attn;
    int32_t reserved;
} aotk_layer;

/* The model graph: what aot-codegen bakes into the generated model.rs as
 * DIMS / TOKEN_EMBD / OUTPUT_NORM / OUTPUT / LAYERS (emit.rs:399-464). */
typedef struct aotk_model_spec {
    aotk_dims dims;
    aotk_flags flags;
    aotk_tensor token_embd, output_norm;
    aotk_tensor output;     /* kind NONE: tied to token_embd (emit.rs:421-424) */
    aotk_tensor rope_freqs; /* kind NONE: no per-dimension factors */
    const aotk_layer *layers; /* dims.n_layer entries */
} aotk_model_spec;

/* ------------------------------------------------------------------------ */
/* Library / device                                                          */
/* ------------------------------------------------------------------------ */

/* Last error of the calling thread (capi.rs:129-141 `aot_last_error`). */
const char *aotk_last_error(void);

/* Select the device and create the library stream. Idempotent. Reads one
 * environment option: AOTK_NO_GRAPH=1 runs the device-side generation loops
 * (aotk_generate_greedy, aotk_generate) as plain stream launches instead of
 * replaying a captured HIP graph per token, so kernel traces list every
 * launch; results are identical either way. */
int aotk_init(int device);

/* Device memory helpers (so C/Rust/Python callers need no HIP headers). */
void *aotk_dev_alloc(size_t bytes);
int aotk_dev_free(void *ptr_dev);
int aotk_h2d(void *dst_dev, const void *src_host, size_t bytes);
int aotk_d2h(void *dst_host, const void *src_dev, size_t bytes);
int aotk_memset(void *dst_dev, int value, size_t bytes);
/* Device-to-device copy on the library stream, synchronous (plumbing with no
 * counterpart in the reference; the benchmark uses it as the known-size copy
 * that calibrates the HBM traffic counters). */
int aotk_d2d(void *dst_dev, const void *src_dev, size_t bytes);
int aotk_sync(void);

/* Bytes per row of `cols` elements (quant.rs:70-73 `Kind::row_bytes`). */
size_t aotk_row_bytes(int kind, size_t cols);

/* ------------------------------------------------------------------------ */
/* Weights in HBM                                                            */
/* ------------------------------------------------------------------------ */

typedef struct aotk_weight aotk_weight;

/* Upload one row-major quantized matrix (`w: &[u8]` of the reference's
 * matvec_* entry points, matvec.rs:358-401) to HBM. The bytes are repacked
 * on the device into the library's aligned plane layout (same byte count). */
aotk_weight *aotk_weight_upload(int kind, const void *bytes_host, size_t rows, size_t cols);
/* Same, from bytes already in device memory (not retained). */
aotk_weight *aotk_weight_from_dev(int kind, const void *bytes_dev, size_t rows, size_t cols);
int aotk_weight_free(aotk_weight *w);

/* Dequantize rows [row0, row0+n_rows) into out_dev (n_rows*cols floats):
 * quant.rs:300-443 (`dequant_row_*`), bit-exact. */
int aotk_dequant_rows(const aotk_weight *w, size_t row0, size_t n_rows, float *out_dev);

/* Reference weight encoders on the device: quantize.rs:282-294
 * (`quantize_row`), applied to every row of x_dev (rows*cols floats);
 * writes rows*row_bytes bytes in the reference (GGUF) layout. Bit-exact. */
int aotk_quantize_rows(int kind, const float *x_dev, size_t rows, size_t cols, void *out_dev);

/* ------------------------------------------------------------------------ */
/* Activation quantizers (quant.rs:231-283)                                  */
/* ------------------------------------------------------------------------ */

/* `quantize_q8_0(x, out)`: n % 32 == 0, out has n/32 blocks. */
int aotk_quantize_q8_0(const float *x_dev, size_t n, aotk_block_q8_0 *out_dev);
/* `quantize_q8_k(x, out)`: n % 256 == 0, out has n/256 blocks. */
int aotk_quantize_q8_k(const float *x_dev, size_t n, aotk_block_q8_k *out_dev);

/* ------------------------------------------------------------------------ */
/* Matrix-vector / matrix-matrix products (matvec.rs:358-583)                */
/* ------------------------------------------------------------------------ */

/* `matvec_<kind>(pool, out, w, x, rows, cols)` with a pre-quantized input:
 * x_dev holds cols/32 aotk_block_q8_0 (Q4_0/Q5_0/Q8_0 weights),
 * cols/256 aotk_block_q8_k (Q4_K/Q5_K/Q6_K) or cols floats (F16/BF16/F32).
 * out_dev[r] = dot(row r, x). Bit-exact with the reference's avx2+f16c
 * kernel set (simd_avx2.rs). */
int aotk_matvec(const aotk_weight *w, const void *x_dev, float *out_dev);

/* Same, with an f32 input vector that is first quantized on the device to
 * the weight's activation format (the generated forward's
 * `quantize_q8_k(&s.xb..); matvec_q4_k(..)` pair, emit.rs:131-140). */
int aotk_matvec_f32(const aotk_weight *w, const float *x_dev, float *out_dev);

/* `matmul_<kind>(pool, out, w, xs, m, rows, cols)` (matvec.rs:524-546):
 * m input vectors back to back in xs_dev (same formats as aotk_matvec),
 * out_dev[i*rows + r]. Bit-identical to m calls of aotk_matvec. */
int aotk_matmul(const aotk_weight *w, const void *xs_dev, size_t m, float *out_dev);

/* Fused products sharing one input, each one launch over the concatenated
 * rows (the reference's single parallel region):
 * aotk_matvec3: `matvec3_q8_k_input` / `matvec3_q8_0_input` (matvec.rs:321-355),
 *   the q/k/v projections: three matrices of one kind and width, rows may
 *   differ; outs[i][r] = dot(row r of ws[i], x).
 * aotk_matvec2: `matvec2_q8_k_input` / `matvec2_q8_0_input` (matvec.rs:403-439),
 *   the gate/up pair: two matrices of one kind and shape.
 * aotk_matmul2: `matmul2_q8_k_input` / `matmul2_q8_0_input` (matvec.rs:569-583),
 *   the batched pair: out_a[i*rows + r], out_b[i*rows + r] for m inputs.
 * Inputs in the formats of aotk_matvec / aotk_matmul; results equal the
 * separate products bit for bit. */
int aotk_matvec3(const aotk_weight *const ws[3], const void *x_dev, float *const outs[3]);
int aotk_matvec2(const aotk_weight *w_a, const aotk_weight *w_b, const void *x_dev, float *out_a, float *out_b);
int aotk_matmul2(const aotk_weight *w_a, const aotk_weight *w_b, const void *xs_dev, size_t m, float *out_a, float *out_b);

/* aotk_matmul without any device allocation. No counterpart in the
 * reference: for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). The Q8_0 / Q8_K
 * inputs are staged in a fixed 4 MiB device array of the library (one per
 * GPU, held until the process ends) instead of the growable scratch; calls
 * whose staging needs more (m * cols * ~2.14 bytes for Q8_K batches of 2 or
 * more, ~1.14 for one input, ~3.13 for Q8_0, e.g. m = 64 at cols up to
 * 28672 for Q8_K) fail with -1. Results equal aotk_matmul's
 * bit for bit. Every call on a GPU shares that GPU's array: calls that
 * overlap on one GPU (from several threads) race. */
int aotk_matmul_noalloc(const aotk_weight *w, const void *xs_dev, size_t m, float *out_dev);

/* ------------------------------------------------------------------------ */
/* Transformer operators (ops.rs)                                            */
/* ------------------------------------------------------------------------ */

/* rmsnorm over m rows of n: ops.rs:7-18, :361-366. */
int aotk_rmsnorm(float *out_dev, const float *x_dev, const float *w_dev, size_t n, size_t m, float eps);
/* rmsnorm_heads in place: ops.rs:74-87. */
int aotk_rmsnorm_heads(float *x_dev, const float *w_dev, size_t n_heads, size_t head_dim, float eps);
/* rope / rope_neox in place over m rows, cs_dev holds m rows of rot_dim
 * interleaved (cos, sin): ops.rs:40-70, :377-391. */
int aotk_rope(float *x_dev, size_t m, size_t n_heads, size_t head_dim, size_t rot_dim, const float *cs_dev, int neox);
/* In-place softmax of n values: ops.rs:98-112. */
int aotk_softmax(float *x_dev, size_t n);
/* h = silu(h)*up / gelu(h)*up: ops.rs:115-134. */
int aotk_silu_mul(float *h_dev, const float *up_dev, size_t n);
int aotk_gelu_mul(float *h_dev, const float *up_dev, size_t n);
/* x += y: ops.rs:145-148. */
int aotk_add(float *x_dev, const float *y_dev, size_t n);
/* Causal GQA attention for m query rows at positions pos0..pos0+m-1 over a
 * [n_layer][ctx][kv_dim] f32 cache: ops.rs:185-218 (`attention`, m == 1) and
 * ops.rs:517-556 (`attention_rows`). window 0 = full attention. */
int aotk_attention(float *out_dev, const float *q_dev, const float *k_cache_dev, const float *v_cache_dev,
                   size_t n_head, size_t n_kv_head, size_t head_dim, size_t ctx, size_t layer,
                   size_t pos0, size_t m, size_t window);
/* First index of the strict maximum: sampler.rs:99-109. */
int aotk_argmax(const float *x_dev, size_t n, uint32_t *out_host);

/* ------------------------------------------------------------------------ */
/* Whole model: the generated forward()/forward_batch() (emit.rs:466-516)    */
/* ------------------------------------------------------------------------ */

typedef struct aotk_model aotk_model;
typedef struct aotk_state aotk_state;

/* Upload the tensor-data blob (the `.incbin` weight section, emit.rs:707-795)
 * to HBM once and build the device tensor table. The spec is copied. */
aotk_model *aotk_model_load(const aotk_model_spec *spec, const void *blob_host, size_t blob_len);
/* Build the model's weights directly in HBM from the synthetic generator
 * (seeded N(0, 0.02)-shaped values, norms 1 + N(0, 0.02)) and the device
 * encoders; the result is byte-identical to encoding the same values with
 * the reference's quantize_row on the host. */
aotk_model *aotk_model_synthetic(const aotk_model_spec *spec, uint64_t seed);
/* Copy the model's blob (reference layout) back to the host. */
int aotk_model_download(const aotk_model *model, void *blob_host, size_t blob_len);
int aotk_model_free(aotk_model *model);
/* HBM bytes read by one decode step's weight matrices (incl. lm-head). */
uint64_t aotk_model_weight_bytes(const aotk_model *model);

/* Activation buffers + KV cache resident in HBM: state.rs:251-355
 * (`State::new(ctx, max_batch)`). The RoPE tables for every position are
 * computed on the host with libm once, exactly like rope_cos_sin
 * (ops.rs:28-34), and uploaded. */
aotk_state *aotk_state_new(aotk_model *model, size_t ctx, size_t max_batch);
int aotk_state_free(aotk_state *state);

/* One decode step (`ForwardFn`, app.rs:32-62; emitted `forward`,
 * emit.rs:466-486). Errors (not panics) on token >= vocab or pos >= ctx. */
int aotk_forward(aotk_state *state, uint32_t token, size_t pos, int want_logits);
/* One batched prompt step of 1..max_batch tokens (`ForwardBatchFn`;
 * emit.rs:491-516); logits of the last token only. */
int aotk_forward_batch(aotk_state *state, const uint32_t *tokens_host, size_t m, size_t pos0, int want_logits);
/* Copy the vocab logits to the host. */
int aotk_logits(aotk_state *state, float *out_host);
/* Greedy token of the current logits (sampler.rs:99-109). */
int aotk_greedy(aotk_state *state, uint32_t *token_out);
/* Greedy generation: starting from the current logits (after the prompt),
 * emit n tokens as app.rs:553-610 does with temperature 0 (sample, then feed
 * back unless it was the last), positions pos, pos+1, ... Writes the n
 * token ids to tokens_host. Device-resident loop: only token ids cross PCIe.
 * The n - 1 forwards must fit the context: pos + n - 1 <= ctx, else -1. */
int aotk_generate_greedy(aotk_state *state, size_t pos, size_t n, uint32_t *tokens_host);
/* KV rows [0, n_pos) of every layer to / from the host, laid out as the
 * reference's cache: [n_layer][n_pos][kv_dim] f32 for K, then the same for V. */
int aotk_kv_download(aotk_state *state, size_t n_pos, float *k_host, float *v_host);
int aotk_kv_upload(aotk_state *state, size_t n_pos, const float *k_host, const float *v_host);
/* Stochastic sampler (sampler.rs:1-114): SamplerConfig field for field
 * (temperature <= 0 selects the arg-max; top_k 0 disables top-k; top_p 1
 * and repeat_penalty 1 disable those) and the xorshift64* stream seeded
 * through splitmix (sampler.rs:32-45, 113-118), kept in device memory.
 * On the device the candidate count min(top_k, vocab) (vocab when top_k is
 * 0) must be at most 1024 when temperature > 0. Candidates of equal scaled
 * logit are ordered by ascending token id (the reference's unstable sort
 * leaves that order open). */
typedef struct aotk_sampler_config {
    float temperature;
    uint32_t top_k;
    float top_p;
    float repeat_penalty;
    uint32_t repeat_last_n;
    uint32_t reserved;
    uint64_t seed;
} aotk_sampler_config;
typedef struct aotk_sampler aotk_sampler;
aotk_sampler *aotk_sampler_new(const aotk_sampler_config *cfg);
int aotk_sampler_free(aotk_sampler *sampler);
/* Sampler::sample on the state's current logits (modified in place by the
 * repetition penalty, sampler.rs:53-60), `recent` = the tokens so far
 * (the last repeat_last_n are penalised). */
int aotk_sample(aotk_state *state, aotk_sampler *sampler, const uint32_t *recent, size_t n_recent, uint32_t *token_out);
/* Replace the state's vocab logits (the `logits: &mut [f32]` argument of
 * Sampler::sample, sampler.rs:49) with a host array. */
int aotk_set_logits(aotk_state *state, const float *logits_host);
/* The generation loop of app.rs:553-610 with a sampler: from the current
 * logits, n tokens at positions pos, pos+1, ... (each fed back except the
 * last), the penalty window running over recent ++ generated. Device-resident
 * like aotk_generate_greedy. */
int aotk_generate(aotk_state *state, aotk_sampler *sampler, size_t pos, size_t n, const uint32_t *recent, size_t n_recent,
                  uint32_t *tokens_out);

/* KV prefix blobs "AOTP" v2 (prefix.rs:15-141; --save-kv / --load-kv and
 * the baked prefix, app.rs:397-489, 631-632).
 * aotk_prefix_save replaces prefix::serialize (prefix.rs:114-141): header,
 * the n_tokens ids, zero padding to 64 bytes, then per layer the K and V rows
 * of positions [0, min(n_cached, n_tokens)). With out == NULL it only stores
 * the blob size in *out_len.
 * aotk_prefix_load replaces Prefix::parse + load_into (prefix.rs:48-108):
 * the checks of parse (magic, version 1 or 2, n_layer and kv_dim of this
 * model, n_tokens > 0, n_cached <= n_tokens, length) fail with -1 where the
 * reference returns None; on success the cached rows go to positions
 * [0, n_cached) of the device cache and the ids to tokens_out (if given). */
int aotk_prefix_save(aotk_state *state, const uint32_t *tokens, size_t n_tokens, size_t n_cached, void *out,
                     size_t out_cap, size_t *out_len);
int aotk_prefix_load(aotk_state *state, const void *blob, size_t len, uint32_t *tokens_out, size_t tokens_cap,
                     size_t *n_tokens, size_t *n_cached);
/* Measurement helper (the reference's #[ignore] bench_ops harness,
 * crates/aot-kernels/tests/metal.rs:459-641): quantizes x_dev once, then
 * launches the matvec of ws[0], ws[1], ... in turn (rotating copies keeps
 * the working set out of the 256 MB Infinity Cache) `iters` times on the
 * library stream, timed with HIP events; writes the mean ms per launch. */
int aotk_time_matvec(const aotk_weight *const *ws, size_t n_w, const float *x_dev, size_t iters, float *ms_per_launch);

/* aotk_time_matvec for a batch: m input vectors of cols floats back to back
 * in xs_dev, quantized once, then the batched product (the prompt kernels
 * for m >= 2) launched `iters` times over ws[0], ws[1], ... in turn. */
int aotk_time_matmul(const aotk_weight *const *ws, size_t n_w, const float *xs_dev, size_t m, size_t iters,
                     float *ms_per_launch);

/* Measurement helper, no reference counterpart (the HBM ceiling that the
 * matvec fractions are read against): `iters` launches of a streaming probe
 * over `bytes` bytes, rotating over the n_bufs device buffers (16-byte
 * aligned): copy == 0 reads bufs[i] (nothing written), copy != 0 copies
 * bufs[i] to bufs[i + 1]; loads_per_lane (1, 2, 4, 8) 16-byte loads in
 * flight per lane, coalesced. Writes the mean ms per launch (HIP events on
 * the library stream). */
int aotk_time_hbm(int copy, int loads_per_lane, void *const *bufs, size_t n_bufs, size_t bytes, size_t iters,
                  float *ms_per_launch);

/* The library's HIP stream (hipStream_t) for callers that time on it. */
void *aotk_stream(void);

#ifdef __cplusplus
}
#endif

#endif /* AOTK_H */
