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
#include "formats.hpp"
#include "internal.hpp"

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

// ss = sum of v*v over n values in LDS, in index order (ops.rs:10-13). Run
// by one thread; the result is broadcast through LDS.
__device__ float seq_sumsq_lds(const float *v, int n, float *bcast) {
    if (threadIdx.x == 0) {
        float ss = 0.0f;
        for (int i = 0; i < n; i += 4) {
            float4 q = *(const float4 *)(v + i);
            ss += q.x * q.x;
            ss += q.y * q.y;
            ss += q.z * q.z;
            ss += q.w * q.w;
        }
        *bcast = ss;
    }
    __syncthreads();
    return *bcast;
}

// Quantize 256 values held 4 per lane (element 4*lane + k) of one wave into
// the Q8_K block `blk` (quant.rs:248-283) and/or the 8 Q8_0 blocks
// 8*blk .. 8*blk+7 (quant.rs:231-245).
__device__ void quant256(const float v[4], int lane, size_t blk, ActQ8K q8k, ActQ8_0 q80) {
    if (q8k.qs) {
        float amax = 0.0f;
        int idx = 0x7fffffff;
        for (int k = 0; k < 4; k++) {
            float a = fabsf(v[k]);
            if (a > amax) { amax = a; idx = lane * 4 + k; }
        }
        for (int m = 1; m < 64; m <<= 1) {
            float oa = shfl_xor(amax, m);
            int oi = shfl_xor(idx, m);
            if (oa > amax || (oa == amax && oi < idx)) { amax = oa; idx = oi; }
        }
        int src_lane = (idx == 0x7fffffff) ? 0 : idx >> 2, sk = idx & 3;
        float c0 = __shfl(v[0], src_lane, 64), c1 = __shfl(v[1], src_lane, 64);
        float c2 = __shfl(v[2], src_lane, 64), c3 = __shfl(v[3], src_lane, 64);
        float max = sk == 0 ? c0 : (sk == 1 ? c1 : (sk == 2 ? c2 : c3));
        uint32_t packed = 0;
        int sum = 0;
        float d = 0.0f;
        if (amax != 0.0f) {
            float iscale = -127.0f / max;
            for (int k = 0; k < 4; k++) {
                int t = round_i(iscale * v[k]);
                t = t > 127 ? 127 : t;
                packed |= (uint32_t)(t & 0xFF) << (8 * k);
                sum += (int8_t)t;
            }
            d = 1.0f / iscale;
        }
        ((uint32_t *)(q8k.qs + blk * 256))[lane] = packed;
        sum += shfl_xor(sum, 1);
        sum += shfl_xor(sum, 2);
        if ((lane & 3) == 0) q8k.bsums[blk * 16 + lane / 4] = (int16_t)sum;
        if (lane == 0) q8k.d[blk] = d;
    }
    if (q80.qs) {
        float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        amax = fmaxf(amax, shfl_xor(amax, 1));
        amax = fmaxf(amax, shfl_xor(amax, 2));
        amax = fmaxf(amax, shfl_xor(amax, 4));
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint32_t packed = 0;
        for (int k = 0; k < 4; k++) packed |= (uint32_t)(clampi(round_i(v[k] * id), -127, 127) & 0xFF) << (8 * k);
        ((uint32_t *)(q80.qs + blk * 256))[lane] = packed;
        if ((lane & 7) == 0) q80.d[blk * 8 + lane / 8] = d;
    }
}

__device__ __forceinline__ ActQ8K q8k_row(ActQ8K a, size_t row, size_t n) {
    if (!a.qs) return a;
    ActQ8K r = a;
    r.qs += row * n;
    r.d += row * (n / 256);
    r.bsums += row * (n / 16);
    return r;
}
__device__ __forceinline__ ActQ8_0 q80_row(ActQ8_0 a, size_t row, size_t n) {
    if (!a.qs) return a;
    ActQ8_0 r = a;
    r.qs += row * n;
    r.d += row * (n / 32);
    return r;
}

// rmsnorm (ops.rs:7-18) of row blockIdx.x, then quantization of the result.
// n % 256 == 0, n <= 8192 (the normalised row is staged in LDS).
__global__ __launch_bounds__(1024) void k_rmsnorm_quant(const float *__restrict__ x, const float *__restrict__ w, int n,
                                                         float eps, RmsOut out) {
    __shared__ __align__(16) float row[8192];
    __shared__ float bc;
    const size_t m = blockIdx.x;
    const float *xr = x + m * n;
    for (int i = threadIdx.x; i < n; i += blockDim.x) row[i] = xr[i];
    __syncthreads();
    float ss = seq_sumsq_lds(row, n, &bc);
    float r = 1.0f / sqrtf(ss / (float)n + eps);
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float v = row[i] * r * w[i];
        row[i] = v;
        if (out.f32) out.f32[m * n + i] = v;
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

void launch_rmsnorm_quant(const float *x, const float *w, size_t n, size_t m, float eps, RmsOut out, hipStream_t s) {
    k_rmsnorm_quant<<<(unsigned)m, 1024, 0, s>>>(x, w, (int)n, eps, out);
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
    size_t total = m * n / 256;
    k_quant_f32<<<(unsigned)((total + 3) / 4), 256, 0, s>>>(x, (int)n, total, out);
}

// silu_mul / gelu_mul (ops.rs:115-134) then quantization; one wave per 256.
__device__ __forceinline__ float silu_f(float v, float b) { return v / (1.0f + aotk_expf(-v)) * b; }
__device__ __forceinline__ float gelu_f(float v) {
    const float k = (float)1.1283791670955126 / (float)1.4142135623730951;
    return 0.5f * v * (1.0f + aotk_tanhf(k * (v + 0.044715f * v * v * v)));
}

__global__ void k_glu_quant(const float *__restrict__ gate, const float *__restrict__ up, int n, size_t total_blk, int gelu,
                            RmsOut out) {
    const int lane = threadIdx.x & 63;
    size_t gb = (size_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (gb >= total_blk) return;
    size_t per = (size_t)n / 256;
    size_t m = gb / per, b = gb % per;
    size_t off = m * n + b * 256 + lane * 4;
    float4 g4 = *(const float4 *)(gate + off);
    float4 u4 = *(const float4 *)(up + off);
    float g[4] = {g4.x, g4.y, g4.z, g4.w}, u[4] = {u4.x, u4.y, u4.z, u4.w};
    float v[4];
    for (int k = 0; k < 4; k++) v[k] = gelu ? gelu_f(g[k]) * u[k] : silu_f(g[k], u[k]);
    if (out.f32) *(float4 *)(out.f32 + off) = make_float4(v[0], v[1], v[2], v[3]);
    quant256(v, lane, b, q8k_row(out.q8k, m, n), q80_row(out.q80, m, n));
}

void launch_glu_quant(const float *gate, const float *up, size_t n, size_t m, int gelu, RmsOut out, hipStream_t s) {
    size_t total = m * n / 256;
    k_glu_quant<<<(unsigned)((total + 3) / 4), 256, 0, s>>>(gate, up, (int)n, total, gelu, out);
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
        __shared__ float bc;
        float ss = seq_sumsq_lds(hv, hd, &bc);
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

template <int HD>
__global__ __launch_bounds__(64) void k_attn_scores(AttnArgs a) {
    __shared__ float sq[ATT_MAX_GQA][HD];
    const int lane = threadIdx.x;
    const int kvh = blockIdx.x, c = blockIdx.y;
    const size_t i = blockIdx.z;
    const int gqa = a.n_head / a.n_kv_head;
    size_t t0, n;
    row_range(a, i, t0, n);
    const size_t start = t0 + (size_t)c * ATT_CH;
    if (start >= n) return;
    const size_t kv = (size_t)a.n_kv_head * HD, q_dim = (size_t)a.n_head * HD;
    for (int h = 0; h < gqa; h++)
        for (int e = lane; e < HD; e += 64) sq[h][e] = a.q[i * q_dim + (size_t)(kvh * gqa + h) * HD + e];
    __syncthreads();
    const size_t t = start + lane;
    if (t >= n) return;
    const float4 *kr = (const float4 *)(a.k_cache + t * kv + (size_t)kvh * HD);
    float acc[ATT_MAX_GQA];
    for (int h = 0; h < gqa; h++) acc[h] = 0.0f;
    for (int d4 = 0; d4 < HD / 4; d4++) {
        float4 k4 = kr[d4];
        for (int h = 0; h < gqa; h++) {
            const float *qq = &sq[h][4 * d4];
            float s = acc[h];
            s += qq[0] * k4.x;
            s += qq[1] * k4.y;
            s += qq[2] * k4.z;
            s += qq[3] * k4.w;
            acc[h] = s;
        }
    }
    for (int h = 0; h < gqa; h++)
        a.prob[(i * a.n_head + (size_t)(kvh * gqa + h)) * a.span + (t - t0)] = acc[h] * a.scale;
}

__global__ __launch_bounds__(256) void k_attn_softmax(AttnArgs a) {
    __shared__ float red[4];
    __shared__ float bc;
    const int h = blockIdx.x;
    const size_t i = blockIdx.y;
    size_t t0, n;
    row_range(a, i, t0, n);
    const int cnt = (int)(n - t0);
    float *p = a.prob + (i * a.n_head + h) * a.span;
    float mx = -INFINITY;
    for (int t = threadIdx.x; t < cnt; t += blockDim.x) mx = fmaxf(mx, p[t]);
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int t = threadIdx.x; t < cnt; t += blockDim.x) p[t] = aotk_expf(p[t] - mx);
    __syncthreads();
    if (threadIdx.x == 0) {
        float sum = 0.0f;
        int t = 0;
        for (; t + 4 <= cnt; t += 4) {
            float4 e = *(const float4 *)(p + t);
            sum += e.x;
            sum += e.y;
            sum += e.z;
            sum += e.w;
        }
        for (; t < cnt; t++) sum += p[t];
        bc = 1.0f / sum;
    }
    __syncthreads();
    const float inv = bc;
    for (int t = threadIdx.x; t < cnt; t += blockDim.x) p[t] = p[t] * inv;
}

// Block = 64 output dims of one head of one row.
__global__ __launch_bounds__(64) void k_attn_out(AttnArgs a) {
    const int hd = a.hd;
    const int per_head = hd / 64;
    const int h = blockIdx.x / per_head, d = (blockIdx.x % per_head) * 64 + threadIdx.x;
    const size_t i = blockIdx.y;
    const int gqa = a.n_head / a.n_kv_head;
    const int kvh = h / gqa;
    size_t t0, n;
    row_range(a, i, t0, n);
    const int cnt = (int)(n - t0);
    const size_t kv = (size_t)a.n_kv_head * hd;
    const float *p = a.prob + (i * a.n_head + h) * a.span;
    const float *vp = a.v_cache + t0 * kv + (size_t)kvh * hd + d;
    float o = 0.0f;
    int t = 0;
    for (; t + 8 <= cnt; t += 8) {
        float v[8], w[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            v[k] = vp[(size_t)(t + k) * kv];
            w[k] = p[t + k];
        }
#pragma unroll
        for (int k = 0; k < 8; k++) o += w[k] * v[k];
    }
    for (; t < cnt; t++) o += p[t] * vp[(size_t)t * kv];
    a.out[i * (size_t)a.n_head * hd + (size_t)h * hd + d] = o;
}

size_t attention_scratch_bytes(size_t n_head, size_t head_dim, size_t ctx, size_t m) {
    (void)head_dim;
    return align_up(m * n_head * align_up(ctx, 4) * 4, 256);
}

void launch_attention(float *out, const float *q, const float *k_cache, const float *v_cache, size_t n_head,
                      size_t n_kv_head, size_t head_dim, size_t ctx_rows, size_t pos0, size_t m, size_t window,
                      const int *pos_dev, float *scratch, size_t scratch_bytes, hipStream_t s) {
    (void)scratch_bytes;
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
    size_t span = window > 0 && window < ctx_rows ? window : ctx_rows;
    dim3 grid((unsigned)n_kv_head, (unsigned)((span + ATT_CH - 1) / ATT_CH), (unsigned)m);
    switch (head_dim) {
    case 64: k_attn_scores<64><<<grid, 64, 0, s>>>(a); break;
    case 128: k_attn_scores<128><<<grid, 64, 0, s>>>(a); break;
    default: k_attn_scores<256><<<grid, 64, 0, s>>>(a); break;
    }
    k_attn_softmax<<<dim3((unsigned)n_head, (unsigned)m), 256, 0, s>>>(a);
    k_attn_out<<<dim3((unsigned)(n_head * head_dim / 64), (unsigned)m), 64, 0, s>>>(a);
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
__global__ __launch_bounds__(1024) void k_rmsnorm_add(float *x, const float *y, const float *w, int n, float eps) {
    __shared__ __align__(16) float row[8192];
    __shared__ float bc;
    const size_t m = blockIdx.x;
    const float *yr = y + m * n;
    float *xr = x + m * n;
    for (int i = threadIdx.x; i < n; i += blockDim.x) row[i] = yr[i];
    __syncthreads();
    float ss = seq_sumsq_lds(row, n, &bc);
    float r = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) xr[i] = xr[i] + row[i] * r * w[i];
}
void launch_rmsnorm_add(float *x, const float *y, const float *w, size_t n, size_t m, float eps, hipStream_t s) {
    k_rmsnorm_add<<<(unsigned)m, 1024, 0, s>>>(x, y, w, (int)n, eps);
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
__global__ __launch_bounds__(1024) void k_softmax(float *x, int n) {
    __shared__ float red[16];
    __shared__ float bc;
    float mx = -INFINITY;
    for (int i = threadIdx.x; i < n; i += blockDim.x) mx = fmaxf(mx, x[i]);
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    float t = (threadIdx.x & 63) < (blockDim.x >> 6) ? red[threadIdx.x & 63] : -INFINITY;
    mx = wave_max(t);
    for (int i = threadIdx.x; i < n; i += blockDim.x) x[i] = aotk_expf(x[i] - mx);
    __syncthreads();
    if (threadIdx.x == 0) {
        float sum = 0.0f;
        for (int i = 0; i < n; i++) sum += x[i];
        bc = 1.0f / sum;
    }
    __syncthreads();
    float inv = bc;
    for (int i = threadIdx.x; i < n; i += blockDim.x) x[i] = x[i] * inv;
}
void launch_softmax(float *x, size_t n, hipStream_t s) { k_softmax<<<1, 1024, 0, s>>>(x, (int)n); }

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
