// internal.hpp - device data layouts and kernel launchers shared by the
// translation units of libaotk.so. Not part of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/aotk.h"

namespace aotk {

constexpr int QK8_0 = 32;
constexpr int QK_K = 256;

__host__ __device__ inline size_t block_size(int kind) {
    switch (kind) {
    case AOTK_F32: case AOTK_F16: case AOTK_BF16: return 1;
    case AOTK_Q4_0: case AOTK_Q5_0: case AOTK_Q8_0: return QK8_0;
    default: return QK_K;
    }
}

__host__ __device__ inline size_t type_size(int kind) {
    switch (kind) {
    case AOTK_F32: return 4;
    case AOTK_F16: case AOTK_BF16: return 2;
    case AOTK_Q4_0: return 18;
    case AOTK_Q5_0: return 22;
    case AOTK_Q8_0: return 34;
    case AOTK_Q4_K: return 144;
    case AOTK_Q5_K: return 176;
    case AOTK_Q6_K: return 210;
    default: return 0;
    }
}

__host__ __device__ inline bool valid_kind(int kind) { return kind >= AOTK_F32 && kind <= AOTK_Q6_K; }
__host__ __device__ inline size_t row_bytes(int kind, size_t cols) { return cols / block_size(kind) * type_size(kind); }

// Activation format consumed by a matrix of `kind` (model.rs:85-91).
enum Act { ACT_F32 = 0, ACT_Q8_0 = 1, ACT_Q8_K = 2 };
__host__ __device__ inline int activation(int kind) {
    switch (kind) {
    case AOTK_Q4_0: case AOTK_Q5_0: case AOTK_Q8_0: return ACT_Q8_0;
    case AOTK_Q4_K: case AOTK_Q5_K: case AOTK_Q6_K: return ACT_Q8_K;
    default: return ACT_F32;
    }
}

__host__ __device__ inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Quantized activation vectors on the device, structure-of-arrays (the
// reference's BlockQ8_K {d, qs[256], bsums[16]} split into planes so every
// load is aligned). One "row" = one input vector of n elements.
struct ActQ8K {
    int8_t *qs;      // [rows][n]
    float *d;        // [rows][n/256]
    int16_t *bsums;  // [rows][n/16]
    // Batches: a second copy of the quants in the matrix-core fragment order
    // (null = none), 4 KB per 16-vector tile and super-block, tiles outer:
    // [tile][super-block][step pair p][k group g][vector v % 16][16 bytes],
    // byte 8h + b holding element 32(2p + h) + 8g + b of the super-block, so
    // that one 16-byte load per lane and step pair gives the A operands of
    // v_mfma_i32_16x16x32_i8 for 16 vectors (see k_mm_kx).
    int8_t *qt;
    int tok;  // vector index of this view's first row
    int nbt;  // super-blocks per vector (n / 256) of the tiled copy
};
struct ActQ8_0 {
    int8_t *qs;     // [rows][n]
    float *d;       // [rows][n/32]
    uint16_t *xh;   // [rows][n] the quants as f16, written for batches of 2 or more (matrix-core products)
};

// Bytes of an activation buffer for `rows` vectors of n elements.
// Batches of 2 or more vectors also hold the tiled copy (whole 16-vector tiles).
inline size_t act_q8k_bytes(size_t n, size_t rows) {
    return align_up(rows * n, 256) + align_up(rows * (n / 256) * 4, 256) + align_up(rows * (n / 16) * 2, 256) +
           (rows >= 2 ? align_up(align_up(rows, 16) * n, 256) : 0);
}
inline ActQ8K act_q8k_view(void *base, size_t n, size_t rows) {
    uint8_t *p = (uint8_t *)base;
    ActQ8K a;
    a.qs = (int8_t *)p;
    p += align_up(rows * n, 256);
    a.d = (float *)p;
    p += align_up(rows * (n / 256) * 4, 256);
    a.bsums = (int16_t *)p;
    p += align_up(rows * (n / 16) * 2, 256);
    a.qt = rows >= 2 ? (int8_t *)p : nullptr;
    a.tok = 0;
    a.nbt = (int)(n / 256);
    return a;
}

// Byte offset in the tiled copy of element e of super-block sb of vector v.
__host__ __device__ inline size_t q8k_tiled_off(size_t v, int sb, int nbt, int e) {
    const int j = e >> 5, g = (e >> 3) & 3;
    return ((v >> 4) * (size_t)nbt + sb) * 4096 + (size_t)((j >> 1) * 1024 + (g * 16 + (int)(v & 15)) * 16 + (j & 1) * 8 + (e & 7));
}
inline size_t act_q8_0_bytes(size_t n, size_t rows) {
    return align_up(rows * n, 256) + align_up(rows * (n / 32) * 4, 256) + align_up(rows * n * 2, 256);
}
inline ActQ8_0 act_q8_0_view(void *base, size_t n, size_t rows) {
    uint8_t *p = (uint8_t *)base;
    ActQ8_0 a;
    a.qs = (int8_t *)p;
    p += align_up(rows * n, 256);
    a.d = (float *)p;
    p += align_up(rows * (n / 32) * 4, 256);
    a.xh = (uint16_t *)p;
    return a;
}

// A weight matrix in HBM in the library's plane layout (same byte count as
// the reference layout; planes are 256-byte aligned):
//   F16, BF16, F32: the reference rows unchanged (row-major);
//   Q4_K, Q5_K: row-major rows, each stored chunk-major: the super-block's
//     bytes [16k, 16k+16) of super-block s at row offset (k*nb + s)*16, so
//     that the 16-byte chunk k of consecutive super-blocks is contiguous;
//   Q6_K: plane0 = the first 208 bytes (ql, qh, scales) of each super-block,
//     chunk-major per row like Q4_K; plane1 = f16 d per super-block;
//   Q8_0: plane0 = 32 quants per block, plane1 = f16 d;
//   Q4_0: plane0 = 16 nibble bytes per block, plane1 = f16 d;
//   Q5_0: plane0 = 16 nibble bytes, plane1 = f16 d, plane2 = u32 qh.
// Block (r, b) of a block plane lives at index r * nb + b.

// Chunk-major row offset of byte `off` of super-block s (K-quants).
__host__ __device__ inline size_t kq_off(size_t off, size_t s, size_t nb) { return ((off >> 4) * nb + s) * 16 + (off & 15); }
struct DevWeight {
    int kind;
    size_t rows, cols, nb;
    uint8_t *base;
    uint8_t *plane[3];
    size_t bytes;  // allocation size
};

size_t weight_dev_bytes(int kind, size_t rows, size_t cols);
void weight_set_planes(DevWeight &w, uint8_t *base);

// ---------------------------------------------------------------- launchers
// All launches go to `s`; none synchronise.

// quant.hip
void launch_repack(const DevWeight &w, const uint8_t *raw, hipStream_t s);
void launch_unpack(const DevWeight &w, uint8_t *raw, hipStream_t s);
void launch_dequant(const DevWeight &w, size_t row0, size_t n_rows, float *out, hipStream_t s);
void launch_encode(int kind, const float *x, size_t rows, size_t cols, uint8_t *raw, hipStream_t s);
void launch_synth(int kind, size_t rows, size_t cols, uint64_t seed, uint32_t tensor_index, int norm, uint8_t *raw,
                  float *scratch, size_t scratch_rows, hipStream_t s);
void launch_quant_q8k(const float *x, size_t n, size_t rows, ActQ8K out, hipStream_t s);
void launch_quant_q8_0(const float *x, size_t n, size_t rows, ActQ8_0 out, hipStream_t s);
void launch_q8k_to_ref(ActQ8K a, size_t n, aotk_block_q8_k *out, hipStream_t s);
void launch_ref_to_q8k(const aotk_block_q8_k *in, size_t n, size_t rows, ActQ8K a, hipStream_t s);
void launch_q8_0_to_ref(ActQ8_0 a, size_t n, aotk_block_q8_0 *out, hipStream_t s);
void launch_ref_to_q8_0(const aotk_block_q8_0 *in, size_t n, size_t rows, ActQ8_0 a, hipStream_t s);

// matvec.hip: y[i*rows + r] (+)= dot(row r, x_i) for m input vectors.
// `add` (may be null) is added to the result (fused residual add).
void launch_matvec(const DevWeight &w, const void *x_act, size_t m, float *y, const float *add, hipStream_t s);
// Up to three matrices sharing kind/cols/input in one launch (q/k/v, gate/up).
// Token sampling (sampler.cpp / sampler.rs); see sampler.hip.
constexpr int SAMP_KMAX = 1024;   // most candidates after top-k on the device
constexpr int SAMP_SLICE = 2048;  // logits per block of the first top-k stage
constexpr int SAMP_MERGE = 8192;  // keys per block of the merge stages
struct SampleArgs {
    float *logits;
    size_t vocab;
    float temperature, top_p, repeat_penalty;
    uint32_t repeat_last_n;
    int k;                // candidates after top-k (temperature > 0)
    uint64_t *rng;        // xorshift64* state
    uint32_t *win;        // tokens so far (penalty window source)
    uint32_t *count;      // entries of win; the pick is appended
    uint32_t *tok_out;    // the picked token
    uint64_t *scratch;    // sampler_scratch_bytes(vocab)
    float *argmax_ws;     // launch_argmax scratch
};
size_t sampler_scratch_bytes(size_t vocab);
void launch_sample(const SampleArgs &p, hipStream_t s);
// One token, the f32 input quantized inside the launch (same bytes as
// launch_quant_f32): K-quant rows of <= 64 super-blocks (to Q8_K), Q8_0 /
// Q4_0 / Q5_0 rows of cols % 256 == 0, cols <= 16384 (to Q8_0).
// Returns false (nothing launched) for other kinds and widths.
bool launch_matvec_quant(const DevWeight &w, const float *x, float *y, const float *add, hipStream_t s);
void launch_matvec_multi(int n, const DevWeight *const ws[], float *const ys[], const void *x_act, size_t m,
                         hipStream_t s);
// Matrices of a Q4_K/Q5_K kind (up to three, e.g. q and k) and one Q6_K
// matrix (e.g. v) with <= 64 super-blocks per row, same input, one launch.
bool matvec_pair_ok(const DevWeight &a, const DevWeight &b);
void launch_matvec_pair(int na, const DevWeight *const wa[], float *const ya[], const DevWeight &wb, float *yb,
                        const void *x_act, size_t m, hipStream_t s);

// ops.hip
struct RmsOut {
    float *f32;     // may be null
    ActQ8K q8k;     // qs null = skip
    ActQ8_0 q80;    // qs null = skip
};
void launch_rmsnorm_quant(const float *x, const float *w, size_t n, size_t m, float eps, RmsOut out, hipStream_t s);
void launch_quant_f32(const float *x, size_t n, size_t m, RmsOut out, hipStream_t s);
// h = act(gate) * up over m rows of n, then optional quantization.
void launch_glu_quant(const float *gate, const float *up, size_t n, size_t m, int gelu, RmsOut out, hipStream_t s);
void launch_embed(const DevWeight &embd, const uint32_t *tokens, size_t m, float scale, int do_scale, float *x, hipStream_t s);
// Per-head post-processing of q/k/v for m rows at positions pos0+i (or *pos_dev
// when pos_dev != null and m == 1): bias, per-head rmsnorm, RoPE, KV store.
struct QkvPost {
    float *q, *k, *v;           // [m][q_dim], [m][kv_dim]
    const float *bq, *bk, *bv;  // may be null
    const float *q_norm, *k_norm;
    const float *cs;            // rope table [ctx][rot_dim]
    float *k_cache, *v_cache;   // layer base
    size_t n_head, n_kv_head, head_dim, rot_dim;
    int neox;
    float eps;
};
void launch_qkv_post(const QkvPost &p, size_t m, size_t pos0, const int *pos_dev, hipStream_t s);
void launch_attention(float *out, const float *q, const float *k_cache, const float *v_cache, size_t n_head,
                      size_t n_kv_head, size_t head_dim, size_t ctx_rows, size_t pos0, size_t m, size_t window,
                      const int *pos_dev, float *scratch, size_t scratch_bytes, hipStream_t s);
size_t attention_scratch_bytes(size_t n_head, size_t head_dim, size_t ctx, size_t m);
// Decode step (one row at *pos_dev or pos0): the q/k/v epilogue of `p`
// (bias, q/k norms, rope, KV store) fused into the scores, then softmax and
// output. Writes out [n_head * head_dim].
void launch_attention_decode(float *out, const QkvPost &p, size_t ctx_rows, size_t pos0, size_t window,
                             const int *pos_dev, float *scratch, hipStream_t s);
void launch_add(float *x, const float *y, size_t n, hipStream_t s);
void launch_rmsnorm_add(float *x, const float *y, const float *w, size_t n, size_t m, float eps, hipStream_t s);
// x += rmsnorm(y) * w_post, then rmsnorm(x) * w_next quantized into `out`.
void launch_rmsnorm_add_quant(float *x, const float *y, const float *w_post, const float *w_next, size_t n, size_t m,
                              float eps, RmsOut out, hipStream_t s);
void launch_argmax(const float *x, size_t n, uint32_t *out_dev, float *scratch, hipStream_t s);
void launch_advance(uint32_t *tok_dev, int *counter_dev, uint32_t *hist, const uint32_t *argmax_dev, hipStream_t s);
void launch_inc(int *p, hipStream_t s);
void launch_softmax(float *x, size_t n, hipStream_t s);
void launch_silu_mul(float *h, const float *up, size_t n, int gelu, hipStream_t s);
void launch_rmsnorm_heads(float *x, const float *w, size_t n_heads, size_t head_dim, float eps, hipStream_t s);
void launch_rope(float *x, size_t m, size_t n_heads, size_t head_dim, size_t rot_dim, const float *cs, int neox,
                 hipStream_t s);

}  // namespace aotk
