// ops.hip - the non-matmul operators of the transformer block on gfx950
// (crates/aot-kernels/src/ops.rs), fused with the activation quantization
// that follows each of them in the generated forward (emit.rs:243-333):
//   rmsnorm -> quantize_q8_k / q8_0, silu_mul / gelu_mul -> quantize,
//   bias + rmsnorm_heads + rope + store_kv in one per-head kernel,
//   GQA decode attention split over position chunks (K/V rows read once),
//   argmax over the vocabulary.
// Every float sum that feeds an activation quantizer runs in the reference's
// sequential order (a different order changes results by an ulp, which flips
// int8 roundings downstream); transcendental functions are the host-libm
// matched aotk_expf / aotk_tanhf. Maxima and integer sums use trees.
#include "device.hpp"
#include "lds_chain.hpp"
#include "formats.hpp"
#include "internal.hpp"
#include "seqsum.hpp"
#include "actfn.hpp"

namespace aotk {

__device__ __forceinline__ float wave_sum(float v) {
    for (int m = 1; m < 64; m <<= 1) v += shfl_xor(v, m);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
    for (int m = 1; m < 64; m <<= 1) v = fmaxf(v, shfl_xor(v, m));
    return v;
}

// Block-wide sum (blockDim.x multiple of 64, at most 1024). Same tree for
// every call with the same blockDim, so results are reproducible.
__device__ float block_sum(float v, float *red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = lane < nw ? red[lane] : 0.0f;
    t = wave_sum(t);
    return t;
}

// Sequential f32 sum of n LDS values in index order, by one thread.
// Plain sums run through lds_chain128 in runs of 128; the rest (and the sums
// of squares) in groups of 32 that alternate between two register sets with
// no copies between them: the reads of the next group are issued before the
// adds of the current one (unconditionally: past the last full group they
// re-read it). v 16-byte aligned.
template <bool SQUARE>
__device__ __forceinline__ float seq_sum_lds(const float *v, int n) {
    float s = 0.0f;
    int i = 0;
    if (!SQUARE)
        for (; i + 128 <= n; i += 128) s = lds_chain128(v + i, s);
    const int nfull = i + (n - i) / 32 * 32;
    auto add = [&](const float4 (&g)[8]) {
#pragma unroll
        for (int k = 0; k < 8; k++) {
            if (SQUARE) {
                s += g[k].x * g[k].x;
                s += g[k].y * g[k].y;
                s += g[k].z * g[k].z;
                s += g[k].w * g[k].w;
            } else {
                s += g[k].x;
                s += g[k].y;
                s += g[k].z;
                s += g[k].w;
            }
        }
    };
    if (nfull > i) {
        const int last = nfull - 32;
        float4 a[8], b[8];
#pragma unroll
        for (int k = 0; k < 8; k++) a[k] = *(const float4 *)(v + i + 4 * k);
        for (;;) {
#pragma unroll
            for (int k = 0; k < 8; k++) b[k] = *(const float4 *)(v + min(i + 32, last) + 4 * k);
            add(a);
            i += 32;
            if (i >= nfull) break;
#pragma unroll
            for (int k = 0; k < 8; k++) a[k] = *(const float4 *)(v + min(i + 32, last) + 4 * k);
            add(b);
            i += 32;
            if (i >= nfull) break;
        }
    }
    for (; i < n; i++) s += SQUARE ? v[i] * v[i] : v[i];
    return s;
}

// The same for v padded with -0.0 up to a multiple of 64 values: whole
// runs of the assembly chain.
__device__ __forceinline__ float seq_sum_lds_pad64(const float *v, int n) {
    const int n64 = (n + 63) & ~63;
    float s = 0.0f;
    int i = 0;
    for (; i + 128 <= n64; i += 128) s = lds_chain128(v + i, s);
    if (i < n64) s = lds_chain64(v + i, s);
    return s;
}

// ss = sum of v*v over n <= 256 values in LDS, in index order
// (ops.rs:10-13), for one wave: the lanes form the squares (each rounded as
// in the sequential loop) into tmp, padded with -0.0 to a run of 64 (neutral
// under round to nearest), then lane 0 adds them in order with the LDS
// chain; the result is returned to every lane.
__device__ __forceinline__ float wave_sumsq_lds(const float *v, float *tmp, int n) {
    const int lane = threadIdx.x & 63;
    const int n64 = (n + 63) & ~63;
    for (int e = lane; e < n64; e += 64) tmp[e] = e < n ? v[e] * v[e] : -0.0f;
    wave_lds_sync();
    float ss = 0.0f;
    if (lane == 0) ss = seq_sum_lds_pad64(tmp, n);
    return __shfl(ss, 0, 64);
}

__device__ __forceinline__ ActQ8K q8k_row(ActQ8K a, size_t row, size_t n) {
    if (!a.qs) return a;
    ActQ8K r = a;
    r.qs += row * n;
    r.d += row * (n / 256);
    r.bsums += row * (n / 16);
    r.tok = (int)row;
    r.nbt = (int)(n / 256);
    return r;
}
__device__ __forceinline__ ActQ8_0 q80_row(ActQ8_0 a, size_t row, size_t n) {
    if (!a.qs) return a;
    ActQ8_0 r = a;
    r.qs += row * n;
    r.d += row * (n / 32);
    if (r.xh) r.xh += row * n;
    return r;
}

// rmsnorm (ops.rs:7-18) of row blockIdx.x, then quantization of the result.
// n % 256 == 0, n <= 8192 (the normalised row is staged in LDS).
#ifndef RMS_TS
#define RMS_TS(i)
#endif
__global__ __launch_bounds__(SEQ_T) void k_rmsnorm_quant(const float *__restrict__ x, const float *__restrict__ w, int n,
                                                         float eps, RmsOut out) {
    __shared__ __align__(16) float row[8192];
    __shared__ float sq[SEQ_PAD_N];
    __shared__ SeqScratch S;
    const size_t m = blockIdx.x;
    const float *xr = x + m * n;
    const int C = seq_chunk(n);
    RMS_TS(0);
    // all of a thread's loads are in flight together (n <= 8 * blockDim.x):
    // the row first, then the norm weights, which stay in flight during the
    // sum (the loads complete in order, so the squares wait for the row only)
    float xv[8], wv[8];
#pragma unroll
    for (int k = 0; k < 8; k++) xv[k] = xr[min((int)threadIdx.x + k * SEQ_T, n - 1)];
#pragma unroll
    for (int k = 0; k < 8; k++) wv[k] = w[min((int)threadIdx.x + k * SEQ_T, n - 1)];
    // the row is needed here, on every path: no load may move into the
    // conditional stores below (and wait there for the norm weights)
#pragma unroll
    for (int k = 0; k < 8; k++) asm volatile("" : "+v"(xv[k]));
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int i = threadIdx.x + k * SEQ_T;
        if (i < n) {
            row[i] = xv[k];
            sq[seq_idx(i, C)] = xv[k] * xv[k];
        }
    }
    __syncthreads();
    RMS_TS(1);
    float ss = exact_seq_sum(sq, n, S);
    RMS_TS(2);
    float r = 1.0f / sqrtf(ss / (float)n + eps);
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int i = threadIdx.x + k * SEQ_T;
        if (i < n) {
            const float v = row[i] * r * wv[k];
            row[i] = v;
            if (out.f32) out.f32[m * n + i] = v;
        }
    }
    RMS_TS(4);
    __syncthreads();
    RMS_TS(5);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    ActQ8K qk = q8k_row(out.q8k, m, n);
    ActQ8_0 q0 = q80_row(out.q80, m, n);
    for (int b = wave; b < n / 256; b += nw) {
        float4 v4 = ((const float4 *)(row + b * 256))[lane];
        float v[4] = {v4.x, v4.y, v4.z, v4.w};
        quant256(v, lane, b, qk, q0);
    }
    RMS_TS(3);
}

// Rows of whole 256-value blocks: thread t holds float4 t (+ 1024 k) of the
// row, so wave w holds the values of quantization blocks w (+ 16 k) in
// quant256's lane order: the normalised row goes from registers straight
// to the quantizer, with no LDS copy and no barrier after the sum.
template <int KF>
__global__ __launch_bounds__(SEQ_T) void k_rmsnorm_quant4(const float *__restrict__ x, const float *__restrict__ w, int n,
                                                         float eps, RmsOut out) {
    __shared__ float sq[SEQ_PAD_N];
    __shared__ SeqScratch S;
    const size_t m = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63;
    const int n4 = n / 4;
    const int C = seq_chunk(n);
    const float4 *xr = (const float4 *)(x + m * n);
    RMS_TS(0);
    float4 xv[KF], wv[KF];
#pragma unroll
    for (int k = 0; k < KF; k++) {
        const int i = tid + k * SEQ_T;
        xv[k] = i < n4 ? xr[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int k = 0; k < KF; k++) {
        const int i = tid + k * SEQ_T;
        wv[k] = i < n4 ? ((const float4 *)w)[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int k = 0; k < KF; k++) {
        const int i = tid + k * SEQ_T;
        if (i < n4) {
            sq[seq_idx(4 * i, C)] = xv[k].x * xv[k].x;
            sq[seq_idx(4 * i + 1, C)] = xv[k].y * xv[k].y;
            sq[seq_idx(4 * i + 2, C)] = xv[k].z * xv[k].z;
            sq[seq_idx(4 * i + 3, C)] = xv[k].w * xv[k].w;
        }
    }
    __syncthreads();
    RMS_TS(1);
    const float ss = exact_seq_sum(sq, n, S);
    RMS_TS(2);
    const float r = 1.0f / sqrtf(ss / (float)n + eps);
    const ActQ8K qk = q8k_row(out.q8k, m, n);
    const ActQ8_0 q0 = q80_row(out.q80, m, n);
#pragma unroll
    for (int k = 0; k < KF; k++) {
        const int i = tid + k * SEQ_T;
        if (i < n4) {  // wave-uniform: n4 is a multiple of 64
            const float v[4] = {xv[k].x * r * wv[k].x, xv[k].y * r * wv[k].y, xv[k].z * r * wv[k].z, xv[k].w * r * wv[k].w};
            if (out.f32) *(float4 *)(out.f32 + m * n + 4 * i) = make_float4(v[0], v[1], v[2], v[3]);
            quant256(v, lane, (size_t)(i >> 6), qk, q0);
        }
    }
    RMS_TS(3);
}

void launch_rmsnorm_quant(const float *x, const float *w, size_t n, size_t m, float eps, RmsOut out, hipStream_t s) {
    if (m < 2) out.q8k.qt = nullptr, out.q80.xh = nullptr;  // the tiled / f16 copies serve batches only
    if (n % 256 == 0 && n <= 4096) k_rmsnorm_quant4<1><<<(unsigned)m, SEQ_T, 0, s>>>(x, w, (int)n, eps, out);
    else if (n % 256 == 0) k_rmsnorm_quant4<2><<<(unsigned)m, SEQ_T, 0, s>>>(x, w, (int)n, eps, out);
    else k_rmsnorm_quant<<<(unsigned)m, SEQ_T, 0, s>>>(x, w, (int)n, eps, out);
}

// Quantize m rows of n floats (n % 256 == 0), one wave per 256 values.
__global__ void k_quant_f32(const float *__restrict__ x, int n, size_t total_blk, RmsOut out) {
    const int lane = threadIdx.x & 63;
    size_t gb = (size_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (gb >= total_blk) return;
    size_t per = (size_t)n / 256;
    size_t m = gb / per, b = gb % per;
    float4 v4 = ((const float4 *)(x + m * n + b * 256))[lane];
    float v[4] = {v4.x, v4.y, v4.z, v4.w};
    quant256(v, lane, b, q8k_row(out.q8k, m, n), q80_row(out.q80, m, n));
}

void launch_quant_f32(const float *x, size_t n, size_t m, RmsOut out, hipStream_t s) {
    if (m < 2) out.q8k.qt = nullptr, out.q80.xh = nullptr;  // the tiled / f16 copies serve batches only
    size_t total = m * n / 256;
    k_quant_f32<<<(unsigned)((total + 3) / 4), 256, 0, s>>>(x, (int)n, total, out);
}

// silu_mul / gelu_mul (ops.rs:115-134) then quantization: block = one
// quantization block of 256 values, one value per thread (the libm-matched
// exp / tanh run once per lane, not four times in a row), then wave 0
// quantizes the block from LDS.
__global__ __launch_bounds__(256) void k_glu_quant(const float *__restrict__ gate, const float *__restrict__ up, int n,
                                                   size_t total_blk, int gelu, RmsOut out) {
    __shared__ __align__(16) float sv[256];
    const size_t gb = blockIdx.x;
    if (gb >= total_blk) return;
    const int t = threadIdx.x;
    const size_t per = (size_t)n / 256;
    const size_t m = gb / per, b = gb % per;
    const size_t off = m * n + b * 256 + t;
    const float g = gate[off], u = up[off];
    const float v = gelu ? gelu_f(g) * u : silu_f(g, u);
    sv[t] = v;
    if (out.f32) out.f32[off] = v;
    __syncthreads();
    if (t < 64) {
        const float4 v4 = ((const float4 *)sv)[t];
        float vv[4] = {v4.x, v4.y, v4.z, v4.w};
        quant256(vv, t, b, q8k_row(out.q8k, m, n), q80_row(out.q80, m, n));
    }
}

void launch_glu_quant(const float *gate, const float *up, size_t n, size_t m, int gelu, RmsOut out, hipStream_t s) {
    if (m < 2) out.q8k.qt = nullptr, out.q80.xh = nullptr;  // the tiled / f16 copies serve batches only
    size_t total = m * n / 256;
    k_glu_quant<<<(unsigned)total, 256, 0, s>>>(gate, up, (int)n, total, gelu, out);
}

// Embedding rows (dequant_row of the token's row, emit.rs:469) [* sqrt(dim)].
template <int KIND>
__global__ void k_embed(WView w, const uint32_t *__restrict__ tokens, size_t cols, float scale, int do_scale, float *x) {
    size_t c = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t i = blockIdx.y;
    if (c >= cols) return;
    float v = dequant_elem<KIND>(w, tokens[i], c);
    if (do_scale) v = v * scale;
    x[i * cols + c] = v;
}

void launch_embed(const DevWeight &embd, const uint32_t *tokens, size_t m, float scale, int do_scale, float *x, hipStream_t s) {
    dim3 grid((unsigned)((embd.cols + 255) / 256), (unsigned)m);
    WView v = view_of(embd);
#define F(K) k_embed<K><<<grid, 256, 0, s>>>(v, tokens, embd.cols, scale, do_scale, x)
    AOTK_KIND_SWITCH(embd.kind, F)
#undef F
}

// ------------------------------------------------ q/k/v per-head epilogue
// One wave per (row, head): bias (ops.rs:89-95), rmsnorm_heads (ops.rs:74-87),
// rope / rope_neox (ops.rs:40-70) with the row's position table, and the
// store_kv copy into the cache (ops.rs:152-157). Heads [0, n_head) are q,
// [n_head, n_head + n_kv_head) are k (+ v).
__global__ __launch_bounds__(64) void k_qkv_post(QkvPost p, size_t pos0, const int *pos_dev) {
    __shared__ __align__(16) float hv[256];
    const int lane = threadIdx.x;
    const size_t i = blockIdx.y;
    const int hh = blockIdx.x;
    const bool is_q = hh < (int)p.n_head;
    const int h = is_q ? hh : hh - (int)p.n_head;
    const int hd = (int)p.head_dim;
    const size_t q_dim = p.n_head * hd, kv_dim = p.n_kv_head * hd;
    const size_t pos = pos_dev ? (size_t)*pos_dev : pos0 + i;
    float *vec = is_q ? p.q + i * q_dim + (size_t)h * hd : p.k + i * kv_dim + (size_t)h * hd;
    const float *bias = is_q ? p.bq : p.bk;
    const float *nw = is_q ? p.q_norm : p.k_norm;
    for (int e = lane; e < hd; e += 64) {
        float v = vec[e];
        if (bias) v = v + bias[(size_t)h * hd + e];
        hv[e] = v;
    }
    __syncthreads();
    if (nw) {
        __shared__ __align__(16) float sqt[256];
        float ss = wave_sumsq_lds(hv, sqt, hd);
        float r = 1.0f / sqrtf(ss / (float)hd + p.eps);
        for (int e = lane; e < hd; e += 64) hv[e] = hv[e] * r * nw[e];
        __syncthreads();
    }
    const float *cs = p.cs + pos * p.rot_dim;
    const int half = (int)p.rot_dim / 2;
    for (int t = lane; t < half; t += 64) {
        float c = cs[2 * t], s = cs[2 * t + 1];
        int a = p.neox ? t : 2 * t, b = p.neox ? t + half : 2 * t + 1;
        float x0 = hv[a], x1 = hv[b];
        hv[a] = x0 * c - x1 * s;
        hv[b] = x0 * s + x1 * c;
    }
    __syncthreads();
    for (int e = lane; e < hd; e += 64) vec[e] = hv[e];
    if (!is_q) {
        float *kc = p.k_cache + pos * kv_dim + (size_t)h * hd;
        float *vc = p.v_cache + pos * kv_dim + (size_t)h * hd;
        const float *vsrc = p.v + i * kv_dim + (size_t)h * hd;
        for (int e = lane; e < hd; e += 64) {
            kc[e] = hv[e];
            float v = vsrc[e];
            if (p.bv) {
                v = v + p.bv[(size_t)h * hd + e];
                ((float *)vsrc)[e] = v;
            }
            vc[e] = v;
        }
    }
}

void launch_qkv_post(const QkvPost &p, size_t m, size_t pos0, const int *pos_dev, hipStream_t s) {
    dim3 grid((unsigned)(p.n_head + p.n_kv_head), (unsigned)m);
    k_qkv_post<<<grid, 64, 0, s>>>(p, pos0, pos_dev);
}

// ----------------------------------------------------------- attention
// Causal GQA attention (ops.rs:185-218 `attention`, :517-556
// `attention_rows`) in the reference's arithmetic order, in three passes:
//   1. scores: one thread per cached position computes q.k sequentially over
//      the head dimension for every query head of the kv group (each K row is
//      read once for the group), times 1/sqrt(hd);
//   2. softmax per (row, head): max, host-libm exp, a sequential sum in
//      position order, multiply by 1/sum (ops.rs:98-112);
//   3. output: one thread per (head, dim) accumulates p_t * v_t in position
//      order (ops.rs:209-215); V rows are read coalesced across dims.
// Scratch: probabilities [m][n_head][span].
constexpr int ATT_CH = 64;
constexpr int ATT_MAX_GQA = 8;

struct AttnArgs {
    float *out;
    const float *q, *k_cache, *v_cache;
    float *prob;
    int n_head, n_kv_head, hd, span;
    size_t pos0, window;
    const int *pos_dev;
    float scale;
};

__device__ __forceinline__ void row_range(const AttnArgs &a, size_t i, size_t &t0, size_t &n) {
    size_t pos = a.pos_dev ? (size_t)*a.pos_dev : a.pos0 + i;
    n = pos + 1;
    t0 = (a.window > 0 && pos + 1 > a.window) ? pos + 1 - a.window : 0;
}

// Scores: block = (kv head, chunk of ATT_CH positions, row), gqa * 64
// threads. The chunk's K rows are staged in LDS (coalesced row loads, row
// stride HD + 1 so that lanes reading one dimension of 64 rows hit 64
// banks); thread (query head of the group, position) then runs its dot
// product sequentially over the head dimension.
template <int HD>
__global__ __launch_bounds__(512) void k_attn_scores(AttnArgs a) {
    constexpr int KS = HD + 1;
    __shared__ float sk[ATT_CH * KS];
    __shared__ __align__(16) float sq[ATT_MAX_GQA][HD];
    const int gqa = a.n_head / a.n_kv_head;
    const int lane = threadIdx.x & 63, hg = threadIdx.x >> 6;
    const int kvh = blockIdx.x, c = blockIdx.y;
    const size_t i = blockIdx.z;
    size_t t0, n;
    row_range(a, i, t0, n);
    const size_t start = t0 + (size_t)c * ATT_CH;
    if (start >= n) return;
    const int rows = (int)min((size_t)ATT_CH, n - start);
    const size_t kv = (size_t)a.n_kv_head * HD, q_dim = (size_t)a.n_head * HD;
    for (int e = lane; e < HD; e += 64) sq[hg][e] = a.q[i * q_dim + (size_t)(kvh * gqa + hg) * HD + e];
    const float *kb = a.k_cache + start * kv + (size_t)kvh * HD;
    constexpr int R4 = HD / 4;
    for (int idx = threadIdx.x; idx < rows * R4; idx += blockDim.x) {
        const int r = idx / R4, c4 = idx % R4;
        const float4 k4 = *(const float4 *)(kb + (size_t)r * kv + 4 * c4);
        float *d = sk + r * KS + 4 * c4;
        d[0] = k4.x;
        d[1] = k4.y;
        d[2] = k4.z;
        d[3] = k4.w;
    }
    __syncthreads();
    if (lane >= rows) return;
    const float *kr = sk + lane * KS;
    const float *qq = sq[hg];
    float s = 0.0f;
#pragma unroll 16
    for (int d = 0; d < HD; d++) s += qq[d] * kr[d];
    a.prob[(i * a.n_head + (size_t)(kvh * gqa + hg)) * a.span + (start + lane - t0)] = s * a.scale;
}

// Prompt scores for ATT_SRB rows per block: block = (kv head, chunk of
// ATT_CH absolute positions, group of ATT_SRB rows), gqa * 64 threads. The
// chunk's K rows are staged once for the group; thread (query head,
// position) runs the rows' dot products side by side, each sequentially over
// the head dimension, and writes those of the rows whose range [t0, n) holds
// the position.
constexpr int ATT_SRB = 4;
template <int HD>
__global__ __launch_bounds__(512) void k_attn_scores_rb(AttnArgs a, int m) {
    constexpr int KS = HD + 4;  // 16-byte rows; lanes reading 16 bytes of 16 rows hit all banks
    __shared__ __align__(16) float sk[ATT_CH * KS];
    __shared__ __align__(16) float sq[ATT_SRB][ATT_MAX_GQA][HD];
    const int gqa = a.n_head / a.n_kv_head;
    const int lane = threadIdx.x & 63, hg = threadIdx.x >> 6;
    const int kvh = blockIdx.x;
    const size_t start = (size_t)blockIdx.y * ATT_CH;
    const int i0 = blockIdx.z * ATT_SRB;
    size_t t0[ATT_SRB], tn[ATT_SRB];
    size_t lo = ~(size_t)0, hi = 0;
#pragma unroll
    for (int r = 0; r < ATT_SRB; r++) {
        row_range(a, (size_t)min(i0 + r, m - 1), t0[r], tn[r]);
        if (i0 + r >= m) tn[r] = t0[r];  // rows past m: empty
        lo = min(lo, t0[r]);
        hi = max(hi, tn[r]);
    }
    if (start >= hi || start + ATT_CH <= lo) return;  // no row has a position here
    const size_t end = min(start + ATT_CH, hi);
    const int rows = (int)(end - start);
    const size_t kv = (size_t)a.n_kv_head * HD, q_dim = (size_t)a.n_head * HD;
    const int nthreads = gqa * 64;
    for (int e = threadIdx.x; e < ATT_SRB * gqa * HD; e += nthreads) {
        const int r = e / (gqa * HD), hh = (e / HD) % gqa, d = e % HD;
        const size_t i = (size_t)min(i0 + r, m - 1);
        sq[r][hh][d] = a.q[i * q_dim + (size_t)(kvh * gqa + hh) * HD + d];
    }
    const float *kb = a.k_cache + start * kv + (size_t)kvh * HD;
    constexpr int R4 = HD / 4;
    for (int idx = threadIdx.x; idx < rows * R4; idx += nthreads) {
        const int r = idx / R4, c4 = idx % R4;
        *(float4 *)(sk + r * KS + 4 * c4) = *(const float4 *)(kb + (size_t)r * kv + 4 * c4);
    }
    __syncthreads();
    if (lane >= rows) return;
    const size_t t = start + lane;
    const float4 *kr = (const float4 *)(sk + lane * KS);
    float sc[ATT_SRB];
#pragma unroll
    for (int r = 0; r < ATT_SRB; r++) sc[r] = 0.0f;
#pragma unroll 2
    for (int d4 = 0; d4 < HD / 4; d4++) {
        const float4 k4 = kr[d4];
#pragma unroll
        for (int r = 0; r < ATT_SRB; r++) {
            const float4 q4 = ((const float4 *)sq[r][hg])[d4];
            sc[r] += q4.x * k4.x;
            sc[r] += q4.y * k4.y;
            sc[r] += q4.z * k4.z;
            sc[r] += q4.w * k4.w;
        }
    }
#pragma unroll
    for (int r = 0; r < ATT_SRB; r++)
        if (t >= t0[r] && t < tn[r])
            a.prob[((size_t)(i0 + r) * a.n_head + (size_t)(kvh * gqa + hg)) * a.span + (t - t0[r])] = sc[r] * a.scale;
}

// Wave-uniform operands through the scalar unit: loads through a pointer in
// the constant address space become s_load (the data is not written during
// the kernel), so a value every lane needs costs no vector load or LDS read.
typedef const float __attribute__((address_space(4))) *att_cfp;
typedef float att_f8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ att_f8 att_sload8(const float *p) { return *(const __attribute__((address_space(4))) att_f8 *)p; }


// Prompt scores: block = (kv head, chunk of 64 absolute positions, group of
// R rows), GQA waves; thread (query head hg = wave, position = lane) runs the
// R rows' dot products side by side, each sequentially over the head
// dimension (s += q[d] * k[d], ops.rs:160-166), then scales them. The q
// values are wave-uniform: scalar loads, 8 dimensions of the R rows at a
// time. The chunk's K rows are staged in LDS 32 dimensions at a time (one
// 16-byte read per lane and 4 dimensions), the next 32 in flight.
constexpr int ATT_KD = 32;  // dimensions per K stage
template <int HD, int GQA, int R>
__global__ __launch_bounds__(64 * GQA) void k_attn_scores_sg(AttnArgs a, int m) {
    constexpr int KS = ATT_KD + 4;
    constexpr int NT = 64 * GQA;
    constexpr int NL = 64 * ATT_KD / 4 / NT;  // float4 loads per thread and stage
    static_assert(NL >= 1, "stage");
    __shared__ __align__(16) float sk[2][64][KS];
    const int tid = threadIdx.x, lane = tid & 63;
    const int hg = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kvh = blockIdx.x;
    const size_t start = (size_t)blockIdx.y * 64;
    const int i0 = blockIdx.z * R;
    size_t t0[R], tn[R];
    size_t lo = ~(size_t)0, hi = 0;
#pragma unroll
    for (int r = 0; r < R; r++) {
        row_range(a, (size_t)min(i0 + r, m - 1), t0[r], tn[r]);
        if (i0 + r >= m) tn[r] = t0[r];  // rows past m: empty
        lo = min(lo, t0[r]);
        hi = max(hi, tn[r]);
    }
    if (start >= hi || start + 64 <= lo) return;  // no row has a position here
    const size_t kv = (size_t)a.n_kv_head * HD, q_dim = (size_t)a.n_head * HD;
    const float *qr[R];
#pragma unroll
    for (int r = 0; r < R; r++) qr[r] = a.q + (size_t)min(i0 + r, m - 1) * q_dim + (size_t)(kvh * GQA + hg) * HD;
    // stage loads: position c / (ATT_KD / 4), dims 4 (c % (ATT_KD / 4)) of the stage (positions past the
    // union's end re-read its last one)
    const float *kb = a.k_cache + (size_t)kvh * HD;
    float4 lk[NL];
    auto fetch = [&](int dc) {
#pragma unroll
        for (int k = 0; k < NL; k++) {
            const int c = tid + NT * k;
            const size_t t = min(start + (size_t)(c / (ATT_KD / 4)), hi - 1);
            lk[k] = *(const float4 *)(kb + t * kv + dc + 4 * (c % (ATT_KD / 4)));
        }
    };
    auto put = [&](int buf) {
#pragma unroll
        for (int k = 0; k < NL; k++) {
            const int c = tid + NT * k;
            *(float4 *)&sk[buf][c / (ATT_KD / 4)][4 * (c % (ATT_KD / 4))] = lk[k];
        }
    };
    fetch(0);
    put(0);
    __syncthreads();
    float sc[R];
#pragma unroll
    for (int r = 0; r < R; r++) sc[r] = 0.0f;
    int buf = 0;
    for (int dc = 0; dc < HD; dc += ATT_KD) {
        const bool more = dc + ATT_KD < HD;
        if (more) fetch(dc + ATT_KD);
#pragma unroll
        for (int d8 = 0; d8 < ATT_KD; d8 += 8) {
            att_f8 q8[R];
#pragma unroll
            for (int r = 0; r < R; r++) q8[r] = att_sload8(qr[r] + dc + d8);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const float4 k4 = *(const float4 *)&sk[buf][lane][d8 + 4 * h];
#pragma unroll
                for (int r = 0; r < R; r++) {
                    sc[r] = sc[r] + q8[r][4 * h] * k4.x;
                    sc[r] = sc[r] + q8[r][4 * h + 1] * k4.y;
                    sc[r] = sc[r] + q8[r][4 * h + 2] * k4.z;
                    sc[r] = sc[r] + q8[r][4 * h + 3] * k4.w;
                }
            }
        }
        if (more) {
            put(buf ^ 1);  // the other buffer was last read before the previous barrier
            __syncthreads();
            buf ^= 1;
        }
    }
    const size_t t = start + lane;
#pragma unroll
    for (int r = 0; r < R; r++)
        if (t >= t0[r] && t < tn[r])
            a.prob[((size_t)(i0 + r) * a.n_head + (size_t)(kvh * GQA + hg)) * a.span + (t - t0[r])] = sc[r] * a.scale;
}

// One wave's share of the q/k/v epilogue for one head vector (decode):
// bias, rmsnorm_heads (sequential sum of squares by lane 0), rope with the
// position's table row; the result is left in `hv` (LDS, HD floats). The
// inputs (the vector, its bias, the norm weights, the rope row) are loaded
// by head_load first, so that loads the caller issues afterwards (the K rows
// of the chunk) do not delay them.
template <int HD>
struct HeadIn {
    static constexpr int NE = (HD + 63) / 64;
    float v[NE], bv[NE], wv[NE];
    float2 cs[NE];
};
template <int HD>
__device__ __forceinline__ void head_load(HeadIn<HD> &in, const float *src, const float *bias, const float *nw,
                                          const float *cs_row, int rot_dim) {
    // unconditional loads (absent inputs read the vector itself, indices
    // past the end repeat the last element): no branch, so no wait, between
    // them
    const int lane = threadIdx.x & 63;
    const int half = rot_dim / 2;
    const float *bp = bias ? bias : src, *wp = nw ? nw : src;
    const float2 *cp = (const float2 *)cs_row;
#pragma unroll
    for (int k = 0; k < HeadIn<HD>::NE; k++) {
        const int e = min(lane + 64 * k, HD - 1);
        in.v[k] = src[e];
        in.bv[k] = bp[e];
        in.wv[k] = wp[e];
        in.cs[k] = cp[max(min(lane + 64 * k, half - 1), 0)];  // (rot_dim > 0 on this path)
    }
}
#ifndef EPI_TS
#define EPI_TS(i)
#endif
template <int HD>
__device__ __forceinline__ void head_post_wave(float *hv, float *tmp, const HeadIn<HD> &in, bool bias, bool norm,
                                               int rot_dim, int neox, float eps) {
    constexpr int NE = HeadIn<HD>::NE;
    const int lane = threadIdx.x & 63;
    const int half = rot_dim / 2;
#pragma unroll
    for (int k = 0; k < NE; k++) {
        const int e = lane + 64 * k;
        if (e < HD) hv[e] = bias ? in.v[k] + in.bv[k] : in.v[k];
    }
    wave_lds_sync();
    EPI_TS(4);
    if (norm) {
        const float ss = wave_sumsq_lds(hv, tmp, HD);
        EPI_TS(5);
        const float r = 1.0f / sqrtf(ss / (float)HD + eps);
#pragma unroll
        for (int k = 0; k < NE; k++) {
            const int e = lane + 64 * k;
            if (e < HD) hv[e] = hv[e] * r * in.wv[k];
        }
        wave_lds_sync();
    }
#pragma unroll
    for (int k = 0; k < NE; k++) {
        const int t = lane + 64 * k;
        if (t < half) {
            const float c = in.cs[k].x, sn = in.cs[k].y;
            const int ia = neox ? t : 2 * t, ib = neox ? t + half : 2 * t + 1;
            const float x0 = hv[ia], x1 = hv[ib];
            hv[ia] = x0 * c - x1 * sn;
            hv[ib] = x0 * sn + x1 * c;
        }
    }
    wave_lds_sync();
    EPI_TS(6);
}

// Decode (one row) scores with the q/k/v epilogue fused in: block = (kv head,
// chunk of ATT_CH positions), (gqa + 1) waves. Waves 0..gqa-1 post-process
// their query head; wave gqa post-processes the new k (and v) of the kv head
// and, in the block whose chunk holds the position, stores both into the
// cache. The chunk's K rows are staged in LDS (the new position's row from
// the post-processed k), then thread (query head, position) runs its dot
// product sequentially over the head dimension.
#ifndef QK_TS
#define QK_TS(i)
#endif
// (head_dim 256: at most 4 query heads per kv head, so that the block's
// 22 float4 of K per thread stay in registers)
constexpr int QKD_MAX_GQA_256 = 4;
template <int HD>
__global__ __launch_bounds__(HD == 256 ? 64 * (QKD_MAX_GQA_256 + 1) : 576) void k_attn_qk_decode(AttnArgs a, QkvPost p) {
    constexpr int KS = HD + 4;  // 16-byte rows; lanes reading 16 bytes of 16 rows hit all banks
    __shared__ __align__(16) float sk[ATT_CH * KS];
    __shared__ __align__(16) float sq[ATT_MAX_GQA + 1][HD];
    const int gqa = a.n_head / a.n_kv_head;
    const int lane = threadIdx.x & 63, hg = threadIdx.x >> 6;
    const int kvh = blockIdx.x, c = blockIdx.y;
    size_t t0, n;
    row_range(a, 0, t0, n);
    const size_t pos = n - 1;
    const size_t start = t0 + (size_t)c * ATT_CH;
    if (start >= n) return;
    const int rows = (int)min((size_t)ATT_CH, n - start);
    const size_t kv = (size_t)a.n_kv_head * HD;
    const float *cs_row = p.cs + pos * p.rot_dim;
    QK_TS(0);
    // the epilogue's inputs first, then the chunk's K rows, which do not
    // depend on it: the first PK float4 of each thread are in flight during
    // the epilogue (the new position's row is filled from the post-processed
    // k below)
    HeadIn<HD> hin;
    if (hg < gqa) {
        const int h = kvh * gqa + hg;
        head_load<HD>(hin, p.q + (size_t)h * HD, p.bq ? p.bq + (size_t)h * HD : nullptr, p.q_norm, cs_row, (int)p.rot_dim);
    } else {
        head_load<HD>(hin, p.k + (size_t)kvh * HD, p.bk ? p.bk + (size_t)kvh * HD : nullptr, p.k_norm, cs_row,
                      (int)p.rot_dim);
    }
    const float *kb = a.k_cache + start * kv + (size_t)kvh * HD;
    constexpr int R4 = HD / 4;
    // every float4 of the chunk a thread loads is in flight at once: up to
    // ATT_CH * HD / 4 over (gqa + 1) * 64 >= 192 threads (gqa >= 2 for
    // HD 256; smaller groups take the loop below for the rest)
    constexpr int PK = HD == 256 ? 22 : 8;
    const int nthreads = (gqa + 1) * 64;
    float4 kpre[PK];
#pragma unroll
    for (int j = 0; j < PK; j++) {
        const int idx = threadIdx.x + j * nthreads;
        const int r = idx / R4, c4 = idx % R4;
        kpre[j] = idx < rows * R4 && start + r != pos ? *(const float4 *)(kb + (size_t)r * kv + 4 * c4)
                                                      : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    // the new position's k and v go to the cache only after the block's
    // barriers (a block barrier waits for the block's outstanding stores)
    const bool owner = hg == gqa && pos >= start && pos < start + ATT_CH;
    float vnew[HD / 64];
    if (owner)
#pragma unroll
        for (int j = 0; j < HD / 64; j++) {
            const int e = lane + 64 * j;
            vnew[j] = p.v[(size_t)kvh * HD + e];
            if (p.bv) vnew[j] = vnew[j] + p.bv[(size_t)kvh * HD + e];
        }
    if (hg < gqa) {
        head_post_wave<HD>(sq[hg], sk + hg * HD, hin, p.bq != nullptr, p.q_norm != nullptr, (int)p.rot_dim, p.neox, p.eps);
    } else {
        float *kn = sq[ATT_MAX_GQA];
        head_post_wave<HD>(kn, sk + gqa * HD, hin, p.bk != nullptr, p.k_norm != nullptr, (int)p.rot_dim, p.neox, p.eps);
    }
    QK_TS(1);
    __syncthreads();  // the epilogue used sk for the squares of the norms
    // K rows of the chunk into LDS (the new position from the post-processed k)
#pragma unroll
    for (int j = 0; j < PK; j++) {
        const int idx = threadIdx.x + j * nthreads;
        if (idx < rows * R4) {
            const int r = idx / R4, c4 = idx % R4;
            *(float4 *)(sk + r * KS + 4 * c4) = kpre[j];
        }
    }
    for (int idx = threadIdx.x + PK * nthreads; idx < rows * R4; idx += nthreads) {
        const int r = idx / R4, c4 = idx % R4;
        float4 k4;
        if (start + r == pos) k4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        else k4 = *(const float4 *)(kb + (size_t)r * kv + 4 * c4);
        *(float4 *)(sk + r * KS + 4 * c4) = k4;
    }
    __syncthreads();
    if (pos >= start && pos < start + ATT_CH) {  // the new row
        const int r = (int)(pos - start);
        for (int e = threadIdx.x; e < HD; e += nthreads) sk[r * KS + e] = sq[ATT_MAX_GQA][e];
        __syncthreads();
    }
    QK_TS(2);
    if (owner) {
        float *kc = p.k_cache + pos * kv + (size_t)kvh * HD;
        float *vc = p.v_cache + pos * kv + (size_t)kvh * HD;
#pragma unroll
        for (int j = 0; j < HD / 64; j++) {
            kc[lane + 64 * j] = sq[ATT_MAX_GQA][lane + 64 * j];
            vc[lane + 64 * j] = vnew[j];
        }
    }
    if (hg >= gqa || lane >= rows) return;
    const float4 *kr = (const float4 *)(sk + lane * KS);
    const float4 *qq = (const float4 *)sq[hg];
    float sc = 0.0f;
#pragma unroll 8
    for (int d4 = 0; d4 < HD / 4; d4++) {
        const float4 k4 = kr[d4], q4 = qq[d4];
        sc += q4.x * k4.x;
        sc += q4.y * k4.y;
        sc += q4.z * k4.z;
        sc += q4.w * k4.w;
    }
    a.prob[(size_t)(kvh * gqa + hg) * a.span + (start + lane - t0)] = sc * a.scale;
    QK_TS(3);
}

// Softmax and output per (row, head, group of SV_DB dims): block of SEQ_T
// threads.
//   softmax (ops.rs:98-112): max, glibc-matched exp, the sequential sum (one
//   thread for short spans, the exact parallel replay for spans of
//   SV_SEQ_MIN..SEQ_MAX_N), multiply by 1/sum; the blocks of one head repeat
//   it identically;
//   output (ops.rs:209-215): chunks of CP positions: all threads form the
//   products p_t * v_t,d into LDS, dim-major (row of dim d: CP products and
//   4 pad floats), with the float4 V loads issued PD chunks ahead; then
//   thread d adds its row in position order (lds_chain) while the others
//   form the next chunk. Sixteen dims per block put 8 blocks on every head
//   (256 for 32 heads); chunks of 384 positions halve the barriers per
//   position against 192.
#ifndef ATT_TS
#define ATT_TS(i)
#endif
#ifndef SV_TS
#define SV_TS(c, i)
#endif
constexpr int ATT_MAX_SPAN = 16384;
constexpr int SV_DB = 16;         // dims per block
constexpr int SV_CP = 384;        // positions per chunk
constexpr int SV_RS = SV_CP + 4;  // floats per dim row of the product buffer
constexpr int SV_BUF = SV_DB * SV_RS;  // floats per product buffer
constexpr int SV_SEQ_MIN = 1024;  // shorter spans are summed by one thread
template <int HD>
__global__ __launch_bounds__(SEQ_T) void k_attn_sv(AttnArgs a) {
    constexpr int DB = SV_DB;
    constexpr int CP = SV_CP;
    __shared__ __align__(16) float e[SEQ_PAD_N > ATT_MAX_SPAN + 64 ? SEQ_PAD_N : ATT_MAX_SPAN + 64];
    // product buffers (+64 floats read past the end by the last groups) / sum scratch
    __shared__ __align__(16) uint8_t ubuf[sizeof(SeqScratch) > (2 * SV_BUF + 64) * 4 ? sizeof(SeqScratch) : (2 * SV_BUF + 64) * 4];
    __shared__ float red[SEQ_T / 64];
    __shared__ float bc;
    __shared__ uint64_t stab[32];  // expf's 2^(i/32) table
    SeqScratch &S = *reinterpret_cast<SeqScratch *>(ubuf);
    float *prod = reinterpret_cast<float *>(ubuf);
    const int tid = threadIdx.x, lane = tid & 63;
    const int h = blockIdx.x / (HD / DB), d0 = (blockIdx.x % (HD / DB)) * DB;
    const size_t i = blockIdx.y;
    const int gqa = a.n_head / a.n_kv_head;
    const int kvh = h / gqa;
    size_t t0, n;
    row_range(a, i, t0, n);
    const int cnt = (int)(n - t0);
    const bool exact = cnt >= SV_SEQ_MIN && cnt <= SEQ_MAX_N;
    const int C = seq_chunk(cnt);
    auto at = [&](int t) { return exact ? seq_idx(t, C) : t; };
    const float *ps = a.prob + (i * a.n_head + h) * a.span;
    const size_t kv = (size_t)a.n_kv_head * HD;
    const float *vb = a.v_cache + t0 * kv + (size_t)kvh * HD + d0;
    constexpr int R4 = DB / 4;
    // wave 0 adds the products; the waves that do not share its SIMD (waves
    // are dealt to the 4 SIMDs in turn) form them, so the dependent adds
    // issue back to back
    constexpr int NPROD = (SEQ_T / 64 - SEQ_T / 256) * 64;
    static_assert(CP == 384, "the output adds of a full chunk run in lds_chain384");
    static_assert(CP * R4 == 2 * NPROD, "two float4 per producer thread per chunk");
    // V loads run PD chunks ahead of the products (a register ring)
    constexpr int PD = 8;
    float4 ring[PD][2];
    const int wv = tid >> 6;
    const int pid = (wv & 3) ? (wv - (wv >> 2) - 1) * 64 + lane : -1;
    auto issue = [&](float4 (&dst)[2], int c) {
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int idx = pid + k * NPROD;
            const int t = c * CP + idx / R4;
            dst[k] = t < cnt ? *(const float4 *)(vb + (size_t)t * kv + 4 * (idx % R4)) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    // the first PE chunks' V loads are in flight through the softmax (more
    // would hold registers the exact sum needs), the rest of the ring after it
    constexpr int PE = 2;
    if (pid >= 0)
#pragma unroll
        for (int j = 0; j < PE; j++) issue(ring[j], j);
    ATT_TS(0);
    // the scores stay in registers (all loads in flight together) through
    // the max; the exps, independent of each other, interleave
    constexpr int SPT = ATT_MAX_SPAN / SEQ_T;  // scores per thread
    exp_table_to_lds(stab);
    float sv[SPT];
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < SPT; k++) {
        const int t = tid + k * SEQ_T;
        sv[k] = t < cnt ? ps[t] : -INFINITY;
    }
#pragma unroll
    for (int k = 0; k < SPT; k++) mx = fmaxf(mx, sv[k]);
    mx = wave_max(mx);
    if (lane == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = wave_max(lane < SEQ_T / 64 ? red[lane] : -INFINITY);
    ATT_TS(1);
#pragma unroll
    for (int k = 0; k < SPT; k++) {
        const int t = tid + k * SEQ_T;
        if (t < cnt) e[at(t)] = aotk_expf_tab(sv[k] - mx, stab);
    }
    // the one-thread sum runs over whole runs of 64: the positions past the
    // span up to the next multiple of 64 hold -0.0, which leaves it unchanged
    if (!exact && tid < 64 && cnt + tid < ((cnt + 63) & ~63)) e[cnt + tid] = -0.0f;
    __syncthreads();
    ATT_TS(2);
    float sum;
    if (exact) {
        sum = exact_seq_sum(e, cnt, S);
    } else {
        if (tid == 0) bc = seq_sum_lds_pad64(e, cnt);
        __syncthreads();
        sum = bc;
    }
    const float inv = 1.0f / sum;
    for (int t = tid; t < cnt; t += SEQ_T) e[at(t)] = e[at(t)] * inv;
    __syncthreads();  // the sum's scratch is reused for the products below
    ATT_TS(3);
    float o = 0.0f;
    const int nch = (cnt + CP - 1) / CP;
    if (pid >= 0)
#pragma unroll
        for (int j = PE; j < PD; j++) issue(ring[j], j);
    for (int c0 = 0; c0 < nch; c0 += PD) {
#pragma unroll
        for (int j = 0; j < PD; j++) {
            const int c = c0 + j;
            if (c < nch) {
                float *buf = prod + (c & 1) * SV_BUF;
                const int base = c * CP;
                const int rows = min(CP, cnt - base);
                if (pid >= 0) {
#pragma unroll
                    for (int k = 0; k < 2; k++) {
                        const int idx = pid + k * NPROD;
                        const int r = idx / R4, d = 4 * (idx % R4);
                        // rows past the span hold -0.0, which leaves any sum unchanged
                        const bool in = r < rows;
                        const float pt = in ? e[at(base + r)] : 0.0f;
                        const float4 v4 = ring[j][k];
                        buf[(d + 0) * SV_RS + r] = in ? pt * v4.x : -0.0f;
                        buf[(d + 1) * SV_RS + r] = in ? pt * v4.y : -0.0f;
                        buf[(d + 2) * SV_RS + r] = in ? pt * v4.z : -0.0f;
                        buf[(d + 3) * SV_RS + r] = in ? pt * v4.w : -0.0f;
                    }
                    issue(ring[j], c + PD);
                }
                SV_TS(c, 0);
                __syncthreads();
                SV_TS(c, 1);
                if (tid < DB) {
                    // the chunk's rows rounded up to 64 (the padding adds -0.0)
                    const float *tp = buf + tid * SV_RS;
                    if (rows > 320) o = lds_chain384(tp, o);
                    else if (rows > 256) o = lds_chain128(tp + 192, lds_chain192(tp, o));
                    else if (rows > 192) o = lds_chain256(tp, o);
                    else if (rows > 128) o = lds_chain192(tp, o);
                    else if (rows > 64) o = lds_chain128(tp, o);
                    else o = lds_chain64(tp, o);
                }
                SV_TS(c, 2);
            }
        }
    }
    ATT_TS(4);
    if (tid < DB) a.out[i * (size_t)a.n_head * HD + (size_t)h * HD + d0 + tid] = o;
}

// Decode attention in one launch for spans of at most AD_MAX_SPAN positions (the
// scores of k_attn_qk_decode and the softmax and output of k_attn_sv): block
// = (head, SV_DB dims) as in k_attn_sv. Wave 0 post-processes the head's q,
// wave 1 the kv head's new k (k_attn_qk_decode's epilogue, the same
// arithmetic), wave 2 loads the new v row; thread t then forms the score of
// position t0 + t (the sequential dot product over the head dimension, the
// new position's k from LDS) straight into registers, and the rest is
// k_attn_sv's code. Every block of the kv head computes the same new k and
// v; the first block of the kv head's first query head stores them into the
// cache, and the products of the new position take v from LDS (its cache
// row is not written yet when other blocks read). One launch fewer per
// layer than the scores + softmax/output pair, for the price of each head's
// scores formed by its HD / SV_DB blocks, each thread reading its position's
// K row (uncoalesced, from L2). Measured against the pair on Llama-3-8B
// decode: 486 -> 504 tok/s at ~140 positions, 480 -> 488 at ~270, 474 ->
// 468 at ~400, 463 -> 430 at ~640; TinyLlama's 38 positions 1080 -> 1159.
// Hence spans of up to 320 positions.
constexpr int AD_MAX_SPAN = 320;
template <int HD>
__global__ __launch_bounds__(SEQ_T) void k_attn_decode1(AttnArgs a, QkvPost p) {
    constexpr int DB = SV_DB;
    constexpr int CP = SV_CP;
    // scores / exps, padded to a run of 64 (spans below SV_SEQ_MIN: the one-thread sum)
    static_assert(AD_MAX_SPAN < SV_SEQ_MIN && AD_MAX_SPAN <= SEQ_T, "one position per thread, the one-thread sum");
    __shared__ __align__(16) float e[AD_MAX_SPAN + 64];
    __shared__ __align__(16) float prod[2 * SV_BUF + 64];  // product buffers (+64 floats read past the end by the last groups)
    __shared__ float red[SEQ_T / 64];
    __shared__ float bc;
    __shared__ uint64_t stab[32];  // expf's 2^(i/32) table
    __shared__ __align__(16) float hq[HD], hk[HD], hv[HD];  // post-processed q, new k, new v
    __shared__ __align__(16) float htmp[2][HD];             // the epilogue's norm scratch
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = tid >> 6;
    const int h = blockIdx.x / (HD / DB), d0 = (blockIdx.x % (HD / DB)) * DB;
    const int gqa = a.n_head / a.n_kv_head;
    const int kvh = h / gqa;
    size_t t0, n;
    row_range(a, 0, t0, n);
    const size_t pos = n - 1;
    const int cnt = (int)(n - t0);
    auto at = [&](int t) { return t; };
    const size_t kv = (size_t)a.n_kv_head * HD;
    const float *vb = a.v_cache + t0 * kv + (size_t)kvh * HD + d0;
    const float *cs_row = p.cs + pos * p.rot_dim;
    // the epilogue's inputs (waves 0 and 1) and the new v row (wave 2)
    HeadIn<HD> hin;
    if (wv == 0)
        head_load<HD>(hin, p.q + (size_t)h * HD, p.bq ? p.bq + (size_t)h * HD : nullptr, p.q_norm, cs_row, (int)p.rot_dim);
    else if (wv == 1)
        head_load<HD>(hin, p.k + (size_t)kvh * HD, p.bk ? p.bk + (size_t)kvh * HD : nullptr, p.k_norm, cs_row,
                      (int)p.rot_dim);
    else if (wv == 2)
        for (int e2 = lane; e2 < HD; e2 += 64) {
            float v = p.v[(size_t)kvh * HD + e2];
            if (p.bv) v = v + p.bv[(size_t)kvh * HD + e2];
            hv[e2] = v;
        }
    constexpr int R4 = DB / 4;
    constexpr int NPROD = (SEQ_T / 64 - SEQ_T / 256) * 64;
    static_assert(CP * R4 == 2 * NPROD, "two float4 per producer thread per chunk");
    constexpr int PD = 8;
    float4 ring[PD][2];
    const int pid = (wv & 3) ? (wv - (wv >> 2) - 1) * 64 + lane : -1;
    auto issue = [&](float4 (&dst)[2], int c) {
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int idx = pid + k * NPROD;
            const int t = c * CP + idx / R4;
            dst[k] = t < cnt ? *(const float4 *)(vb + (size_t)t * kv + 4 * (idx % R4)) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    };
    constexpr int PE = 2;
    if (pid >= 0)
#pragma unroll
        for (int j = 0; j < PE; j++) issue(ring[j], j);
    exp_table_to_lds(stab);
    if (wv == 0) head_post_wave<HD>(hq, htmp[0], hin, p.bq != nullptr, p.q_norm != nullptr, (int)p.rot_dim, p.neox, p.eps);
    else if (wv == 1) head_post_wave<HD>(hk, htmp[1], hin, p.bk != nullptr, p.k_norm != nullptr, (int)p.rot_dim, p.neox, p.eps);
    __syncthreads();
    // the new position's k and v into the cache: one block per kv head
    if (blockIdx.x == (unsigned)(kvh * gqa * (HD / DB)) && wv == 1) {
        float *kc = p.k_cache + pos * kv + (size_t)kvh * HD;
        float *vc = p.v_cache + pos * kv + (size_t)kvh * HD;
        for (int e2 = lane; e2 < HD; e2 += 64) {
            kc[e2] = hk[e2];
            vc[e2] = hv[e2];
        }
    }
    // the scores: thread t, position t0 + t (k_attn_qk_decode's dot product)
    float sv0 = -INFINITY;
    if (tid < cnt) {
        const float4 *kr = t0 + tid == pos ? (const float4 *)hk : (const float4 *)(a.k_cache + (t0 + tid) * kv + (size_t)kvh * HD);
        const float4 *qq = (const float4 *)hq;
        float sc = 0.0f;
#pragma unroll 8
        for (int d4 = 0; d4 < HD / 4; d4++) {
            const float4 k4 = kr[d4], q4 = qq[d4];
            sc += q4.x * k4.x;
            sc += q4.y * k4.y;
            sc += q4.z * k4.z;
            sc += q4.w * k4.w;
        }
        sv0 = sc * a.scale;
    }
    float mx = wave_max(sv0);
    if (lane == 0) red[wv] = mx;
    __syncthreads();
    mx = wave_max(lane < SEQ_T / 64 ? red[lane] : -INFINITY);
    if (tid < cnt) e[at(tid)] = aotk_expf_tab(sv0 - mx, stab);
    if (tid < 64 && cnt + tid < ((cnt + 63) & ~63)) e[cnt + tid] = -0.0f;
    __syncthreads();
    if (tid == 0) bc = seq_sum_lds_pad64(e, cnt);
    __syncthreads();
    const float sum = bc;
    const float inv = 1.0f / sum;
    for (int t = tid; t < cnt; t += SEQ_T) e[at(t)] = e[at(t)] * inv;
    __syncthreads();  // the sum's scratch is reused for the products below
    float o = 0.0f;
    const int nch = (cnt + CP - 1) / CP;
    if (pid >= 0)
#pragma unroll
        for (int j = PE; j < PD; j++) issue(ring[j], j);
    for (int c0 = 0; c0 < nch; c0 += PD) {
#pragma unroll
        for (int j = 0; j < PD; j++) {
            const int c = c0 + j;
            if (c < nch) {
                float *buf = prod + (c & 1) * SV_BUF;
                const int base = c * CP;
                const int rows = min(CP, cnt - base);
                if (pid >= 0) {
#pragma unroll
                    for (int k = 0; k < 2; k++) {
                        const int idx = pid + k * NPROD;
                        const int r = idx / R4, d = 4 * (idx % R4);
                        const bool in = r < rows;
                        const float pt = in ? e[at(base + r)] : 0.0f;
                        // the new position's v from LDS (its cache row may not be written yet)
                        const float4 v4 = base + r == cnt - 1 ? *(const float4 *)(hv + d0 + d) : ring[j][k];
                        buf[(d + 0) * SV_RS + r] = in ? pt * v4.x : -0.0f;
                        buf[(d + 1) * SV_RS + r] = in ? pt * v4.y : -0.0f;
                        buf[(d + 2) * SV_RS + r] = in ? pt * v4.z : -0.0f;
                        buf[(d + 3) * SV_RS + r] = in ? pt * v4.w : -0.0f;
                    }
                    issue(ring[j], c + PD);
                }
                __syncthreads();
                if (tid < DB) {
                    const float *tp = buf + tid * SV_RS;
                    if (rows > 320) o = lds_chain384(tp, o);
                    else if (rows > 256) o = lds_chain128(tp + 192, lds_chain192(tp, o));
                    else if (rows > 192) o = lds_chain256(tp, o);
                    else if (rows > 128) o = lds_chain192(tp, o);
                    else if (rows > 64) o = lds_chain128(tp, o);
                    else o = lds_chain64(tp, o);
                }
            }
        }
    }
    if (tid < DB) a.out[(size_t)h * HD + d0 + tid] = o;
}

// Batched rows (prompt chunks), spans up to ATT_MAX_SPAN: the same softmax
// and output, with the serial chains spread over lanes instead of blocks.
//   k_attn_softmax_rows: one wave per (row, head) for spans up to
//   ATT_ROWS_MAX: max, glibc-matched exp into LDS, the sequential sum by
//   lane 0, then p = e * (1 / sum) written back over the scores; longer
//   spans: k_attn_softmax_rows_x, a block per (row, head).
//   k_attn_out_rows: one wave per (head, 64-dim slice, ATT_RB rows: 2 at
//   head_dim <= 128, 1 at 256); lane d keeps the ATT_RB sums of dim d and
//   adds p_t * v_t,d in position order;
//   V rows are read straight from the cache (256 B per wave per position),
//   the probabilities with wave-uniform loads.
constexpr int ATT_ROWS_MAX = 2048;  // spans of the one-wave softmax (four waves per block)

template <int NW, int CAP>
__global__ __launch_bounds__(64 * NW) void k_attn_softmax_rows(AttnArgs a, int m) {
    __shared__ __align__(16) float e[NW][CAP];
    __shared__ uint64_t stab[32];  // expf's 2^(i/32) table (an LDS read per lookup)
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int pair = blockIdx.x * NW + w;
    exp_table_to_lds(stab);
    __syncthreads();
    if (pair >= m * a.n_head) return;
    const int i = pair / a.n_head, h = pair % a.n_head;
    size_t t0, n;
    row_range(a, i, t0, n);
    const int cnt = (int)(n - t0);
    float *ps = a.prob + ((size_t)i * a.n_head + h) * a.span;
    float *ew = e[w];
    // every score load of the lane in flight together (a loop that stores
    // each one as it arrives waits for the loads one at a time)
    constexpr int VPL = CAP / 64;
    float v[VPL];
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < VPL; k++) {
        const int t = lane + 64 * k;
        v[k] = t < cnt ? ps[t] : -INFINITY;
    }
#pragma unroll
    for (int k = 0; k < VPL; k++) mx = fmaxf(mx, v[k]);
    mx = wave_max(mx);
#pragma unroll
    for (int k = 0; k < VPL; k++) {
        const int t = lane + 64 * k;
        if (t < cnt) {
            v[k] = aotk_expf_tab(v[k] - mx, stab);
            ew[t] = v[k];
        }
    }
    if (cnt + lane < ((cnt + 63) & ~63)) ew[cnt + lane] = -0.0f;  // neutral padding to a run of 64
    wave_lds_sync();
    float sum = 0.0f;
    if (lane == 0) sum = seq_sum_lds_pad64(ew, cnt);
    const float inv = 1.0f / readlane_f(sum, 0);
#pragma unroll
    for (int k = 0; k < VPL; k++) {
        const int t = lane + 64 * k;
        if (t < cnt) ps[t] = v[k] * inv;
    }
}

template <int HD, int ATT_RB, int GS = 32>
__global__ __launch_bounds__(256) void k_attn_out_rows(AttnArgs a, int m) {
    static_assert(ATT_RB == 4 || ATT_RB == 2 || ATT_RB == 1, "one float4 / float2 / float of p per position");
    static_assert((GS == 32 || GS == 64) && GS * ATT_RB <= 128, "positions per group: the p slot holds 128 floats");
    __shared__ float4 sPr[4][32];
    constexpr int NS = HD / 64;
    const int lane = threadIdx.x & 63;
    const int wv = threadIdx.x >> 6;
    const int task = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const int slice = task % NS, h = (task / NS) % a.n_head, rg = task / (NS * a.n_head);
    if (rg * ATT_RB >= m) return;
    const int gqa = a.n_head / a.n_kv_head, kvh = h / gqa;
    const size_t kv = (size_t)a.n_kv_head * HD;
    const int d = slice * 64 + lane;
    int row[ATT_RB];
    size_t t0[ATT_RB], tn[ATT_RB];
    const float *pr[ATT_RB];
    size_t lo = ~(size_t)0, hi = 0, alo = 0, ahi = ~(size_t)0;
#pragma unroll
    for (int r = 0; r < ATT_RB; r++) {
        row[r] = min(rg * ATT_RB + r, m - 1);  // rows past m repeat the last one, unstored
        row_range(a, row[r], t0[r], tn[r]);
        pr[r] = a.prob + ((size_t)row[r] * a.n_head + h) * a.span - t0[r];
        lo = min(lo, t0[r]);
        hi = max(hi, tn[r]);
        alo = max(alo, t0[r]);
        ahi = min(ahi, tn[r]);
    }
    const float *vb = a.v_cache + (size_t)kvh * HD + d;
    float o[ATT_RB];
#pragma unroll
    for (int r = 0; r < ATT_RB; r++) o[r] = 0.0f;
    auto step_if = [&](size_t t) {
        const float v = vb[t * kv];
#pragma unroll
        for (int r = 0; r < ATT_RB; r++)
            if (t >= t0[r] && t < tn[r]) o[r] += pr[r][t] * v;
    };
    if (alo >= ahi) {  // no position common to all rows
        for (size_t t = lo; t < hi; t++) step_if(t);
    } else {
        for (size_t t = lo; t < alo; t++) step_if(t);
        // groups of 32 positions in two register sets (A, B), each loaded one
        // group ahead of its use: V with one load per position, p with one
        // load per row (lane k holds position k), written to this wave's LDS
        // slot as [position][row] so that one broadcast 16-byte read gives
        // the four rows' p of a position
        size_t t = alo;
        float va[GS], pa[ATT_RB], vbb[GS], pb[ATT_RB];
        float4 *sp = sPr[wv];
        auto load = [&](float (&v)[GS], float (&pv)[ATT_RB], size_t c) {
#pragma unroll
            for (int k = 0; k < GS; k++) v[k] = vb[(c + k) * kv];
#pragma unroll
            for (int r = 0; r < ATT_RB; r++) pv[r] = pr[r][c + (lane & (GS - 1))];
        };
        auto use = [&](const float (&v)[GS], const float (&pv)[ATT_RB]) {
            if (ATT_RB == 4) {
                if (lane < GS) sp[lane] = make_float4(pv[0], pv[ATT_RB > 1 ? 1 : 0], pv[ATT_RB > 2 ? 2 : 0], pv[ATT_RB > 3 ? 3 : 0]);
            } else if (ATT_RB == 2) {
                if (lane < GS) ((float2 *)sp)[lane] = make_float2(pv[0], pv[ATT_RB > 1 ? 1 : 0]);
            } else {
                if (lane < GS) ((float *)sp)[lane] = pv[0];
            }
            wave_lds_sync();
#pragma unroll
            for (int k = 0; k < GS; k++) {
                if (ATT_RB == 4) {
                    const float4 p4 = sp[k];
                    o[0] += p4.x * v[k];
                    o[ATT_RB > 1 ? 1 : 0] += p4.y * v[k];
                    o[ATT_RB > 2 ? 2 : 0] += p4.z * v[k];
                    o[ATT_RB > 3 ? 3 : 0] += p4.w * v[k];
                } else if (ATT_RB == 2) {
                    const float2 p2 = ((const float2 *)sp)[k];
                    o[0] += p2.x * v[k];
                    o[ATT_RB > 1 ? 1 : 0] += p2.y * v[k];
                } else {
                    o[0] += ((const float *)sp)[k] * v[k];
                }
            }
            wave_lds_sync();
        };
        if (t + GS <= ahi) load(va, pa, t);
        while (t + GS <= ahi) {
            const bool more = t + 2 * GS <= ahi;
            if (more) load(vbb, pb, t + GS);
            use(va, pa);
            t += GS;
            if (!more) break;
            const bool more2 = t + 2 * GS <= ahi;
            if (more2) load(va, pa, t + GS);
            use(vbb, pb);
            t += GS;
            if (!more2) break;
        }
        for (; t < ahi; t++) {
            const float v = vb[t * kv];
#pragma unroll
            for (int r = 0; r < ATT_RB; r++) o[r] += pr[r][t] * v;
        }
        for (t = ahi; t < hi; t++) step_if(t);
    }
#pragma unroll
    for (int r = 0; r < ATT_RB; r++)
        if (rg * ATT_RB + r < m) a.out[(size_t)row[r] * a.n_head * HD + (size_t)h * HD + d] = o[r];
}

// The same for rows of more than ATT_ROWS_MAX positions: a block of SEQ_T
// threads per (row, head), the scores held in registers through the max,
// the exps with the 2^(i/32) table in LDS, the exact parallel replay of the
// sequential sum (one wave's single-thread sum of 4096 terms took ~100 us).
template <int CAP>
__global__ __launch_bounds__(SEQ_T) void k_attn_softmax_rows_x(AttnArgs a, int m) {
    __shared__ __align__(16) float e[CAP + SEQ_T + 32];
    __shared__ SeqScratch S;
    __shared__ float red[SEQ_T / 64];
    __shared__ uint64_t stab[32];
    constexpr int SPT = CAP / SEQ_T;
    const int tid = threadIdx.x, lane = tid & 63;
    const int i = blockIdx.x / a.n_head, h = blockIdx.x % a.n_head;
    size_t t0, n;
    row_range(a, i, t0, n);
    const int cnt = (int)(n - t0);
    float *ps = a.prob + ((size_t)i * a.n_head + h) * a.span;
    exp_table_to_lds(stab);
    float sv[SPT];
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < SPT; k++) {
        const int t = tid + k * SEQ_T;
        sv[k] = t < cnt ? ps[t] : -INFINITY;
        mx = fmaxf(mx, sv[k]);
    }
    mx = wave_max(mx);
    if (lane == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = wave_max(lane < SEQ_T / 64 ? red[lane] : -INFINITY);
    const int C = seq_chunk(cnt);
#pragma unroll
    for (int k = 0; k < SPT; k++) {
        const int t = tid + k * SEQ_T;
        if (t < cnt) {
            sv[k] = aotk_expf_tab(sv[k] - mx, stab);
            e[seq_idx(t, C)] = sv[k];
        }
    }
    __syncthreads();
    const float inv = 1.0f / exact_seq_sum(e, cnt, S);
#pragma unroll
    for (int k = 0; k < SPT; k++) {
        const int t = tid + k * SEQ_T;
        if (t < cnt) ps[t] = sv[k] * inv;
    }
}

// The same on 256 threads per (row, head) (spans up to CAP <= 8192): the
// prompt runs m x n_head of these at once, so the issue count of the exact
// sum matters more than its latency.
template <int CAP>
__global__ __launch_bounds__(256) void k_attn_softmax_rows_q(AttnArgs a, int m) {
    constexpr int T = 256;
    __shared__ __align__(16) float e[CAP + T + 32];
    __shared__ SeqScratch S;
    __shared__ float red[T / 64];
    __shared__ uint64_t stab[32];
    constexpr int SPT = CAP / T;
    const int tid = threadIdx.x, lane = tid & 63;
    const int i = blockIdx.x / a.n_head, h = blockIdx.x % a.n_head;
    size_t t0, n;
    row_range(a, i, t0, n);
    const int cnt = (int)(n - t0);
    float *ps = a.prob + ((size_t)i * a.n_head + h) * a.span;
    exp_table_to_lds(stab);
    float sv[SPT];
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < SPT; k++) {
        const int t = tid + k * T;
        sv[k] = t < cnt ? ps[t] : -INFINITY;
        mx = fmaxf(mx, sv[k]);
    }
    mx = wave_max(mx);
    if (lane == 0) red[tid >> 6] = mx;
    __syncthreads();
    mx = wave_max(lane < T / 64 ? red[lane] : -INFINITY);
    const int C = seq_chunk_of(cnt, T);
#pragma unroll
    for (int k = 0; k < SPT; k++) {
        const int t = tid + k * T;
        if (t < cnt) {
            sv[k] = aotk_expf_tab(sv[k] - mx, stab);
            e[seq_idx(t, C)] = sv[k];
        }
    }
    __syncthreads();
    const float inv = 1.0f / exact_seq_sum256(e, cnt, S);
#pragma unroll
    for (int k = 0; k < SPT; k++) {
        const int t = tid + k * T;
        if (t < cnt) ps[t] = sv[k] * inv;
    }
}


static void launch_rows(const AttnArgs &a, size_t head_dim, size_t m, size_t longest, hipStream_t s) {
    const unsigned pairs = (unsigned)(m * a.n_head);
    // many (row, head) pairs: the 256-thread exact sum for spans past 1024
    // (measured at 64 rows x 32 heads: 4096 positions 64 -> 51 us); few
    // pairs (8 heads at 8192 positions: 27 against 34 us) keep the
    // 1024-thread form
    const bool many = pairs >= 1024;
    if (many && longest > 1024 && longest <= 4096) k_attn_softmax_rows_q<4096><<<pairs, 256, 0, s>>>(a, (int)m);
    else if (many && longest > 4096 && longest <= 8192) k_attn_softmax_rows_q<8192><<<pairs, 256, 0, s>>>(a, (int)m);
    else if (longest <= (size_t)ATT_ROWS_MAX) k_attn_softmax_rows<4, ATT_ROWS_MAX><<<(pairs + 3) / 4, 256, 0, s>>>(a, (int)m);
    else if (longest <= 8192) k_attn_softmax_rows_x<8192><<<pairs, SEQ_T, 0, s>>>(a, (int)m);
    else k_attn_softmax_rows_x<ATT_MAX_SPAN><<<pairs, SEQ_T, 0, s>>>(a, (int)m);
    // rows per wave (measured at 64 rows against 4: head_dim 128 two rows,
    // 4096 positions 160 -> 127 us, 512 positions 25 -> 21 us; head_dim 256
    // one row, 8192 positions 297 -> 213 us, a 1024 window 47 -> 30 us)
    const int RB = head_dim == 256 ? 1 : 2;
    // V loads 64 positions ahead instead of 32 for long spans (measured:
    // Qwen3 4096 positions 126 -> 118 us, Gemma-3 8192 206 -> 194 us,
    // a 1024 window 29 -> 28 us; 512 positions 21 -> 23 us)
    const bool deep = longest >= 1024;
    const size_t tasks = (m + RB - 1) / RB * a.n_head * (head_dim / 64);
    const unsigned g = (unsigned)((tasks + 3) / 4);
    switch (head_dim) {
    case 64: k_attn_out_rows<64, 2><<<g, 256, 0, s>>>(a, (int)m); break;
    case 128:
        if (deep) k_attn_out_rows<128, 2, 64><<<g, 256, 0, s>>>(a, (int)m);
        else k_attn_out_rows<128, 2><<<g, 256, 0, s>>>(a, (int)m);
        break;
    default:
        if (deep) k_attn_out_rows<256, 1, 64><<<g, 256, 0, s>>>(a, (int)m);
        else k_attn_out_rows<256, 1><<<g, 256, 0, s>>>(a, (int)m);
        break;
    }
}

static void launch_sv(const AttnArgs &a, size_t head_dim, size_t m, hipStream_t s) {
    dim3 g((unsigned)(a.n_head * (head_dim / SV_DB)), (unsigned)m);
    switch (head_dim) {
    case 64: k_attn_sv<64><<<g, SEQ_T, 0, s>>>(a); break;
    case 128: k_attn_sv<128><<<g, SEQ_T, 0, s>>>(a); break;
    default: k_attn_sv<256><<<g, SEQ_T, 0, s>>>(a); break;
    }
}

size_t attention_scratch_bytes(size_t n_head, size_t head_dim, size_t ctx, size_t m) {
    (void)head_dim;
    return align_up(m * n_head * align_up(ctx, 4) * 4, 256);
}

static AttnArgs attn_args(float *out, const float *q, const float *k_cache, const float *v_cache, size_t n_head,
                          size_t n_kv_head, size_t head_dim, size_t ctx_rows, size_t pos0, size_t window,
                          const int *pos_dev, float *scratch) {
    AttnArgs a;
    a.out = out;
    a.q = q;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.prob = scratch;
    a.span = (int)align_up(ctx_rows, 4);
    a.n_head = (int)n_head;
    a.n_kv_head = (int)n_kv_head;
    a.hd = (int)head_dim;
    a.pos0 = pos0;
    a.window = window;
    a.pos_dev = pos_dev;
    a.scale = 1.0f / sqrtf((float)head_dim);
    return a;
}

void launch_attention(float *out, const float *q, const float *k_cache, const float *v_cache, size_t n_head,
                      size_t n_kv_head, size_t head_dim, size_t ctx_rows, size_t pos0, size_t m, size_t window,
                      const int *pos_dev, float *scratch, size_t scratch_bytes, hipStream_t s) {
    (void)scratch_bytes;
    AttnArgs a = attn_args(out, q, k_cache, v_cache, n_head, n_kv_head, head_dim, ctx_rows, pos0, window, pos_dev,
                           scratch);
    size_t span = window > 0 && window < ctx_rows ? window : ctx_rows;
    dim3 grid((unsigned)n_kv_head, (unsigned)((span + ATT_CH - 1) / ATT_CH), (unsigned)m);
    const unsigned threads = (unsigned)(64 * (n_head / n_kv_head));
    const size_t gqa_ratio = n_head / n_kv_head;
    if (m > 1 && !pos_dev && head_dim == 256 &&
        (gqa_ratio == 1 || gqa_ratio == 2 || gqa_ratio == 4 || gqa_ratio == 8)) {
        // head_dim 256: rows batched per block, q through the scalar unit
        // (measured at 64 rows: 8192 positions 839 -> 188 us, a 1024 window
        // 68 -> 43 us; at head_dim 128 the per-row-group kernel below stays
        // ahead, 107 against 114 us at 4096 positions)
        const size_t hi = pos0 + m;  // the last row's end
        const int gqa = (int)(n_head / n_kv_head);
        dim3 g4((unsigned)n_kv_head, (unsigned)((hi + 63) / 64), (unsigned)((m + 3) / 4));
        switch (gqa) {
        case 1: k_attn_scores_sg<256, 1, 4><<<g4, 64, 0, s>>>(a, (int)m); break;
        case 2: k_attn_scores_sg<256, 2, 4><<<g4, 128, 0, s>>>(a, (int)m); break;
        case 4: k_attn_scores_sg<256, 4, 4><<<g4, 256, 0, s>>>(a, (int)m); break;
        case 8: k_attn_scores_sg<256, 8, 4><<<g4, 512, 0, s>>>(a, (int)m); break;
        }
    } else if (m > 1 && !pos_dev && head_dim <= 128) {
        // several rows per block over absolute position chunks
        const size_t hi = pos0 + m;  // the last row's end
        dim3 g((unsigned)n_kv_head, (unsigned)((hi + ATT_CH - 1) / ATT_CH), (unsigned)((m + ATT_SRB - 1) / ATT_SRB));
        if (head_dim == 64) k_attn_scores_rb<64><<<g, threads, 0, s>>>(a, (int)m);
        else k_attn_scores_rb<128><<<g, threads, 0, s>>>(a, (int)m);
    } else {
        switch (head_dim) {
        case 64: k_attn_scores<64><<<grid, threads, 0, s>>>(a); break;
        case 128: k_attn_scores<128><<<grid, threads, 0, s>>>(a); break;
        default: k_attn_scores<256><<<grid, threads, 0, s>>>(a); break;
        }
    }
    // the longest row spans min(pos0 + m, window) positions
    const size_t longest = window > 0 && window < pos0 + m ? window : pos0 + m;
    if (m > 1 && !pos_dev && longest <= (size_t)ATT_MAX_SPAN)
        launch_rows(a, head_dim, m, longest, s);
    else
        launch_sv(a, head_dim, m, s);
}

void launch_attention_decode(float *out, const QkvPost &p, size_t ctx_rows, size_t pos0, size_t window,
                             const int *pos_dev, float *scratch, hipStream_t s) {
    AttnArgs a = attn_args(out, p.q, p.k_cache, p.v_cache, p.n_head, p.n_kv_head, p.head_dim, ctx_rows, pos0, window,
                           pos_dev, scratch);
    size_t span = window > 0 && window < ctx_rows ? window : ctx_rows;
    if (span <= (size_t)AD_MAX_SPAN) {  // short spans: scores, softmax and output in one launch
        const dim3 g1((unsigned)(p.n_head * (p.head_dim / SV_DB)), 1);
        switch (p.head_dim) {
        case 64: k_attn_decode1<64><<<g1, SEQ_T, 0, s>>>(a, p); break;
        case 128: k_attn_decode1<128><<<g1, SEQ_T, 0, s>>>(a, p); break;
        default: k_attn_decode1<256><<<g1, SEQ_T, 0, s>>>(a, p); break;
        }
        return;
    }
    dim3 grid((unsigned)p.n_kv_head, (unsigned)((span + ATT_CH - 1) / ATT_CH), 1);
    const unsigned threads = (unsigned)(64 * (p.n_head / p.n_kv_head + 1));
    switch (p.head_dim) {
    case 64: k_attn_qk_decode<64><<<grid, threads, 0, s>>>(a, p); break;
    case 128: k_attn_qk_decode<128><<<grid, threads, 0, s>>>(a, p); break;
    default: k_attn_qk_decode<256><<<grid, threads, 0, s>>>(a, p); break;
    }
    launch_sv(a, p.head_dim, 1, s);
}

// ------------------------------------------------------------ elementwise

__global__ void k_add(float *x, const float *y, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = x[i] + y[i];
}
void launch_add(float *x, const float *y, size_t n, hipStream_t s) {
    k_add<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(x, y, n);
}

// Gemma post-norm join: x += rmsnorm(y) (emit.rs:320-324).
__global__ __launch_bounds__(SEQ_T) void k_rmsnorm_add(float *x, const float *y, const float *w, int n, float eps) {
    __shared__ float sq[SEQ_PAD_N];
    __shared__ SeqScratch S;
    const size_t m = blockIdx.x;
    const float *yr = y + m * n;
    float *xr = x + m * n;
    const int C = seq_chunk(n);
    // every load (y, and x and w for the update) is issued before the sum, y
    // first: the loads complete in order, so the squares wait for y only
    float yv[8], xv[8], wv[8];
#pragma unroll
    for (int k = 0; k < 8; k++) yv[k] = yr[min((int)threadIdx.x + k * SEQ_T, n - 1)];
#pragma unroll
    for (int k = 0; k < 8; k++) xv[k] = xr[min((int)threadIdx.x + k * SEQ_T, n - 1)];
#pragma unroll
    for (int k = 0; k < 8; k++) wv[k] = w[min((int)threadIdx.x + k * SEQ_T, n - 1)];
    // y is needed here, on every path: no load may move into the conditional
    // stores below (and wait there for x and w)
#pragma unroll
    for (int k = 0; k < 8; k++) asm volatile("" : "+v"(yv[k]));
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int i = threadIdx.x + k * SEQ_T;
        if (i < n) sq[seq_idx(i, C)] = yv[k] * yv[k];
    }
    __syncthreads();
    RMS_TS(1);
    float ss = exact_seq_sum(sq, n, S);
    RMS_TS(2);
    float r = 1.0f / sqrtf(ss / (float)n + eps);
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int i = threadIdx.x + k * SEQ_T;
        if (i < n) xr[i] = xv[k] + yv[k] * r * wv[k];
    }
}
// Gemma: the post-norm join x += rmsnorm(y) (emit.rs:320-324) and the next
// rmsnorm of x with its quantization (the following block's input), in one
// launch: the updated row stays in registers between the two exact sums.
__global__ __launch_bounds__(SEQ_T) void k_rmsnorm_add_quant(float *x, const float *y, const float *w_post,
                                                             const float *w_next, int n, float eps, RmsOut out) {
    __shared__ __align__(16) float row[8192];
    __shared__ float sq[SEQ_PAD_N];
    __shared__ SeqScratch S;
    const size_t m = blockIdx.x;
    const float *yr = y + m * n;
    float *xr = x + m * n;
    const int C = seq_chunk(n);
    float yv[8], xv[8], wv[8], wn[8];
#pragma unroll
    for (int k = 0; k < 8; k++) yv[k] = yr[min((int)threadIdx.x + k * SEQ_T, n - 1)];
#pragma unroll
    for (int k = 0; k < 8; k++) xv[k] = xr[min((int)threadIdx.x + k * SEQ_T, n - 1)];
#pragma unroll
    for (int k = 0; k < 8; k++) wv[k] = w_post[min((int)threadIdx.x + k * SEQ_T, n - 1)];
#pragma unroll
    for (int k = 0; k < 8; k++) wn[k] = w_next[min((int)threadIdx.x + k * SEQ_T, n - 1)];
#pragma unroll
    for (int k = 0; k < 8; k++) asm volatile("" : "+v"(yv[k]));
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int i = threadIdx.x + k * SEQ_T;
        if (i < n) sq[seq_idx(i, C)] = yv[k] * yv[k];
    }
    __syncthreads();
    const float ss = exact_seq_sum(sq, n, S);
    const float r = 1.0f / sqrtf(ss / (float)n + eps);
    // x += y * r * w (as k_rmsnorm_add), then the squares of the new x
    // (exact_seq_sum's closing barrier orders these writes after its reads)
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int i = threadIdx.x + k * SEQ_T;
        if (i < n) {
            const float v = xv[k] + yv[k] * r * wv[k];
            xv[k] = v;
            row[i] = v;
            sq[seq_idx(i, C)] = v * v;
        }
    }
    __syncthreads();
    const float ss2 = exact_seq_sum(sq, n, S);
    const float r2 = 1.0f / sqrtf(ss2 / (float)n + eps);
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const int i = threadIdx.x + k * SEQ_T;
        if (i < n) {
            xr[i] = xv[k];  // stored after the sums (see k_rmsnorm_add_quant4)
            const float v = row[i] * r2 * wn[k];
            row[i] = v;
            if (out.f32) out.f32[m * n + i] = v;
        }
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    ActQ8K qk = q8k_row(out.q8k, m, n);
    ActQ8_0 q0 = q80_row(out.q80, m, n);
    for (int b = wave; b < n / 256; b += nw) {
        float4 v4 = ((const float4 *)(row + b * 256))[lane];
        float v[4] = {v4.x, v4.y, v4.z, v4.w};
        quant256(v, lane, b, qk, q0);
    }
}

// The same for rows of whole 256-blocks, float4 per thread as in
// k_rmsnorm_quant4 (the joined row quantized from registers).
template <int KF>
__global__ __launch_bounds__(SEQ_T) void k_rmsnorm_add_quant4(float *x, const float *y, const float *w_post,
                                                              const float *w_next, int n, float eps, RmsOut out) {
    __shared__ float sq[SEQ_PAD_N];
    __shared__ SeqScratch S;
    const size_t m = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63;
    const int n4 = n / 4;
    const int C = seq_chunk(n);
    float4 *xr = (float4 *)(x + m * n);
    const float4 *yr = (const float4 *)(y + m * n);
    float4 yv[KF], xv[KF], wv[KF], wn[KF];
    const float4 z = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int k = 0; k < KF; k++) yv[k] = tid + k * SEQ_T < n4 ? yr[tid + k * SEQ_T] : z;
#pragma unroll
    for (int k = 0; k < KF; k++) xv[k] = tid + k * SEQ_T < n4 ? xr[tid + k * SEQ_T] : z;
#pragma unroll
    for (int k = 0; k < KF; k++) wv[k] = tid + k * SEQ_T < n4 ? ((const float4 *)w_post)[tid + k * SEQ_T] : z;
#pragma unroll
    for (int k = 0; k < KF; k++) wn[k] = tid + k * SEQ_T < n4 ? ((const float4 *)w_next)[tid + k * SEQ_T] : z;
    auto squares = [&](const float4 &v, int i) {
        sq[seq_idx(4 * i, C)] = v.x * v.x;
        sq[seq_idx(4 * i + 1, C)] = v.y * v.y;
        sq[seq_idx(4 * i + 2, C)] = v.z * v.z;
        sq[seq_idx(4 * i + 3, C)] = v.w * v.w;
    };
#pragma unroll
    for (int k = 0; k < KF; k++)
        if (tid + k * SEQ_T < n4) squares(yv[k], tid + k * SEQ_T);
    __syncthreads();
    const float ss = exact_seq_sum(sq, n, S);
    const float r = 1.0f / sqrtf(ss / (float)n + eps);
    // x += y * r * w (as k_rmsnorm_add), then the squares of the new x
    // (exact_seq_sum's closing barrier orders these writes after its reads)
#pragma unroll
    for (int k = 0; k < KF; k++) {
        const int i = tid + k * SEQ_T;
        if (i < n4) {
            float4 v;
            v.x = xv[k].x + yv[k].x * r * wv[k].x;
            v.y = xv[k].y + yv[k].y * r * wv[k].y;
            v.z = xv[k].z + yv[k].z * r * wv[k].z;
            v.w = xv[k].w + yv[k].w * r * wv[k].w;
            xv[k] = v;
            squares(v, i);
        }
    }
    __syncthreads();
    const float ss2 = exact_seq_sum(sq, n, S);
    const float r2 = 1.0f / sqrtf(ss2 / (float)n + eps);
    const ActQ8K qk = q8k_row(out.q8k, m, n);
    const ActQ8_0 q0 = q80_row(out.q80, m, n);
    // the new x is stored only now: a store in flight would hold up every
    // barrier of the second sum (a block barrier waits for the block's
    // outstanding memory operations)
#pragma unroll
    for (int k = 0; k < KF; k++) {
        const int i = tid + k * SEQ_T;
        if (i < n4) xr[i] = xv[k];
    }
#pragma unroll
    for (int k = 0; k < KF; k++) {
        const int i = tid + k * SEQ_T;
        if (i < n4) {  // wave-uniform: n4 is a multiple of 64
            const float v[4] = {xv[k].x * r2 * wn[k].x, xv[k].y * r2 * wn[k].y, xv[k].z * r2 * wn[k].z, xv[k].w * r2 * wn[k].w};
            if (out.f32) *(float4 *)(out.f32 + m * n + 4 * i) = make_float4(v[0], v[1], v[2], v[3]);
            quant256(v, lane, (size_t)(i >> 6), qk, q0);
        }
    }
}

void launch_rmsnorm_add_quant(float *x, const float *y, const float *w_post, const float *w_next, size_t n, size_t m,
                              float eps, RmsOut out, hipStream_t s) {
    if (m < 2) out.q8k.qt = nullptr, out.q80.xh = nullptr;  // the tiled / f16 copies serve batches only
    if (n % 256 == 0 && n <= 4096) k_rmsnorm_add_quant4<1><<<(unsigned)m, SEQ_T, 0, s>>>(x, y, w_post, w_next, (int)n, eps, out);
    else if (n % 256 == 0) k_rmsnorm_add_quant4<2><<<(unsigned)m, SEQ_T, 0, s>>>(x, y, w_post, w_next, (int)n, eps, out);
    else k_rmsnorm_add_quant<<<(unsigned)m, SEQ_T, 0, s>>>(x, y, w_post, w_next, (int)n, eps, out);
}

void launch_rmsnorm_add(float *x, const float *y, const float *w, size_t n, size_t m, float eps, hipStream_t s) {
    k_rmsnorm_add<<<(unsigned)m, SEQ_T, 0, s>>>(x, y, w, (int)n, eps);
}

__global__ void k_silu_mul(float *h, const float *up, size_t n, int gelu) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    h[i] = gelu ? gelu_f(h[i]) * up[i] : silu_f(h[i], up[i]);
}
void launch_silu_mul(float *h, const float *up, size_t n, int gelu, hipStream_t s) {
    k_silu_mul<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(h, up, n, gelu);
}

// softmax (ops.rs:98-112) of one vector: max, exp, sequential sum, scale.
__global__ __launch_bounds__(SEQ_T) void k_softmax(float *x, int n) {
    __shared__ float red[16];
    __shared__ float bc;
    __shared__ float ev[SEQ_PAD_N];
    __shared__ SeqScratch S;
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < n; i += blockDim.x) mx = fmaxf(mx, x[i]);
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    float t = (threadIdx.x & 63) < (blockDim.x >> 6) ? red[threadIdx.x & 63] : -INFINITY;
    mx = wave_max(t);
    for (int i = threadIdx.x; i < n; i += blockDim.x) x[i] = aotk_expf(x[i] - mx);
    __syncthreads();
    float sum;
    if (n <= SEQ_MAX_N) {
        const int C = seq_chunk(n);
        for (int i = threadIdx.x; i < n; i += blockDim.x) ev[seq_idx(i, C)] = x[i];
        __syncthreads();
        sum = exact_seq_sum(ev, n, S);
    } else {
        if (threadIdx.x == 0) {
            float t = 0.0f;
            for (int i = 0; i < n; i++) t += x[i];
            bc = t;
        }
        __syncthreads();
        sum = bc;
    }
    float inv = 1.0f / sum;
    for (int i = threadIdx.x; i < n; i += blockDim.x) x[i] = x[i] * inv;
}
void launch_softmax(float *x, size_t n, hipStream_t s) { k_softmax<<<1, SEQ_T, 0, s>>>(x, (int)n); }

void launch_rmsnorm_heads(float *x, const float *w, size_t n_heads, size_t head_dim, float eps, hipStream_t s) {
    QkvPost p = {};
    p.q = x;
    p.q_norm = w;
    p.n_head = n_heads;
    p.n_kv_head = 0;
    p.head_dim = head_dim;
    p.rot_dim = 0;
    p.eps = eps;
    static float dummy_cs[2];
    (void)dummy_cs;
    p.cs = x;  // unused with rot_dim == 0
    launch_qkv_post(p, 1, 0, nullptr, s);
}

void launch_rope(float *x, size_t m, size_t n_heads, size_t head_dim, size_t rot_dim, const float *cs, int neox,
                 hipStream_t s) {
    // positions 0..m-1 index the m rows of the table
    QkvPost p = {};
    p.q = x;
    p.n_head = n_heads;
    p.n_kv_head = 0;
    p.head_dim = head_dim;
    p.rot_dim = rot_dim;
    p.cs = cs;
    p.neox = neox;
    launch_qkv_post(p, m, 0, nullptr, s);
}

// ----------------------------------------------------------------- argmax
// First index of the strict maximum (sampler.rs:99-109): -inf and NaN never
// win; an empty / all -inf input gives 0.
__device__ __forceinline__ void amax_merge(float &bv, uint32_t &bi, float v, uint32_t i) {
    if (v > bv || (v == bv && i < bi)) { bv = v; bi = i; }
}

__global__ __launch_bounds__(1024) void k_argmax_part(const float *x, size_t n, size_t per, float *pv, uint32_t *pi) {
    __shared__ float sv[16];
    __shared__ uint32_t si[16];
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    size_t s0 = blockIdx.x * per, s1 = s0 + per < n ? s0 + per : n;
    for (size_t i = s0 + threadIdx.x; i < s1; i += blockDim.x) {
        float v = x[i];
        if (v > -INFINITY) amax_merge(bv, bi, v, (uint32_t)i);
    }
    for (int m = 1; m < 64; m <<= 1) {
        float ov = shfl_xor(bv, m);
        uint32_t oi = shfl_xor(bi, m);
        amax_merge(bv, bi, ov, oi);
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); w++) amax_merge(bv, bi, sv[w], si[w]);
        pv[blockIdx.x] = bv;
        pi[blockIdx.x] = bi;
    }
}

__global__ void k_argmax_final(const float *pv, const uint32_t *pi, int np, uint32_t *out) {
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (int i = threadIdx.x; i < np; i += 64) amax_merge(bv, bi, pv[i], pi[i]);
    for (int m = 1; m < 64; m <<= 1) {
        float ov = shfl_xor(bv, m);
        uint32_t oi = shfl_xor(bi, m);
        amax_merge(bv, bi, ov, oi);
    }
    if (threadIdx.x == 0) *out = bi == 0xFFFFFFFFu ? 0u : bi;
}

void launch_argmax(const float *x, size_t n, uint32_t *out_dev, float *scratch, hipStream_t s) {
    const int np = 128;
    size_t per = (n + np - 1) / np;
    float *pv = scratch;
    uint32_t *pi = (uint32_t *)(scratch + np);
    k_argmax_part<<<np, 1024, 0, s>>>(x, n, per, pv, pi);
    k_argmax_final<<<1, 64, 0, s>>>(pv, pi, np, out_dev);
}

// Device-resident greedy loop: next token = argmax, recorded at hist[counter++].
__global__ void k_advance(uint32_t *tok, int *pos, uint32_t *hist, const uint32_t *am) {
    uint32_t t = *am;
    int p = *pos;
    *tok = t;
    if (hist) hist[p] = t;
    *pos = p + 1;
}
void launch_advance(uint32_t *tok_dev, int *counter_dev, uint32_t *hist, const uint32_t *argmax_dev, hipStream_t s) {
    k_advance<<<1, 1, 0, s>>>(tok_dev, counter_dev, hist, argmax_dev);
}

__global__ void k_inc(int *p) { *p = *p + 1; }
void launch_inc(int *p, hipStream_t s) { k_inc<<<1, 1, 0, s>>>(p); }

}  // namespace aotk
