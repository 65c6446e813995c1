// quant.hip - weight formats on the device: repacking into the aligned plane
// layout, dequantization (quant.rs:300-443), the reference weight encoders
// (quantize.rs:16-294), the synthetic generator, and the activation
// quantizers quantize_q8_0 / quantize_q8_k (quant.rs:231-283).
#include "device.hpp"
#include "internal.hpp"
#include "formats.hpp"

namespace aotk {

// ------------------------------------------------------------------ layout

size_t weight_dev_bytes(int kind, size_t rows, size_t cols) {
    size_t nb = cols / block_size(kind);
    size_t n = rows * nb;
    switch (kind) {
    case AOTK_Q6_K: return align_up(n * 208, 256) + align_up(n * 2, 256);
    case AOTK_Q8_0: return align_up(n * 32, 256) + align_up(n * 2, 256);
    case AOTK_Q4_0: return align_up(n * 16, 256) + align_up(n * 2, 256);
    case AOTK_Q5_0: return align_up(n * 16, 256) + align_up(n * 2, 256) + align_up(n * 4, 256);
    default: return align_up(rows * row_bytes(kind, cols), 256);
    }
}

void weight_set_planes(DevWeight &w, uint8_t *base) {
    w.nb = w.cols / block_size(w.kind);
    size_t n = w.rows * w.nb;
    w.base = base;
    w.plane[0] = base;
    w.plane[1] = w.plane[2] = nullptr;
    switch (w.kind) {
    case AOTK_Q6_K: w.plane[1] = base + align_up(n * 208, 256); break;
    case AOTK_Q8_0: w.plane[1] = base + align_up(n * 32, 256); break;
    case AOTK_Q4_0: w.plane[1] = base + align_up(n * 16, 256); break;
    case AOTK_Q5_0:
        w.plane[1] = base + align_up(n * 16, 256);
        w.plane[2] = w.plane[1] + align_up(n * 2, 256);
        break;
    default: break;
    }
    w.bytes = weight_dev_bytes(w.kind, w.rows, w.cols);
}

// Planar formats: how a reference block of TS bytes maps onto the planes.
// Q4_K / Q5_K: chunk-major row in p0
// Q6_K: [0,208) -> chunk-major row in p0, [208,210) -> p1 (2/blk)
// Q8_0: [0,2) -> p1, [2,34) -> p0 (32/blk)
// Q4_0: [0,2) -> p1, [2,18) -> p0 (16/blk)
// Q5_0: [0,2) -> p1, [2,6) -> p2 (4/blk), [6,22) -> p0 (16/blk)
template <int KIND>
struct Planar;
template <> struct Planar<AOTK_Q4_K> { static constexpr int TS = 144; };
template <> struct Planar<AOTK_Q5_K> { static constexpr int TS = 176; };
template <> struct Planar<AOTK_Q6_K> { static constexpr int TS = 210; };
template <> struct Planar<AOTK_Q8_0> { static constexpr int TS = 34; };
template <> struct Planar<AOTK_Q4_0> { static constexpr int TS = 18; };
template <> struct Planar<AOTK_Q5_0> { static constexpr int TS = 22; };

template <int KIND>
__device__ __forceinline__ uint8_t *plane_byte(size_t blk, size_t nb, int off, uint8_t *p0, uint8_t *p1, uint8_t *p2) {
    if (KIND == AOTK_Q4_K || KIND == AOTK_Q5_K) {
        const size_t r = blk / nb, sb = blk % nb;
        return p0 + r * nb * Planar<KIND>::TS + kq_off(off, sb, nb);
    }
    if (KIND == AOTK_Q6_K) {
        const size_t r = blk / nb, sb = blk % nb;
        return off < 208 ? p0 + r * nb * 208 + kq_off(off, sb, nb) : p1 + blk * 2 + (off - 208);
    }
    if (KIND == AOTK_Q8_0) return off < 2 ? p1 + blk * 2 + off : p0 + blk * 32 + (off - 2);
    if (KIND == AOTK_Q4_0) return off < 2 ? p1 + blk * 2 + off : p0 + blk * 16 + (off - 2);
    return off < 2 ? p1 + blk * 2 + off : (off < 6 ? p2 + blk * 4 + (off - 2) : p0 + blk * 16 + (off - 6));
}

template <int KIND, bool TO_PLANES>
__global__ void k_repack(size_t nblk, size_t nb, uint8_t *raw, uint8_t *p0, uint8_t *p1, uint8_t *p2) {
    size_t blk = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= nblk) return;
    constexpr int TS = Planar<KIND>::TS;
    uint8_t *src = raw + blk * TS;  // rows are contiguous: block index is global
    for (int off = 0; off < TS; off++) {
        uint8_t *pb = plane_byte<KIND>(blk, nb, off, p0, p1, p2);
        if (TO_PLANES) *pb = src[off];
        else src[off] = *pb;
    }
}

template <bool TO_PLANES>
static void repack_common(const DevWeight &w, uint8_t *raw, hipStream_t s) {
    size_t nblk = w.rows * w.nb;
    size_t bytes = w.rows * row_bytes(w.kind, w.cols);
    unsigned grid = (unsigned)((nblk + 255) / 256);
    switch (w.kind) {
#define AOTK_REPACK(K) \
    case K: k_repack<K, TO_PLANES><<<grid, 256, 0, s>>>(nblk, w.nb, raw, w.plane[0], w.plane[1], w.plane[2]); break;
        AOTK_REPACK(AOTK_Q4_K)
        AOTK_REPACK(AOTK_Q5_K)
        AOTK_REPACK(AOTK_Q6_K)
        AOTK_REPACK(AOTK_Q8_0)
        AOTK_REPACK(AOTK_Q4_0)
        AOTK_REPACK(AOTK_Q5_0)
#undef AOTK_REPACK
    default:
        if (TO_PLANES) (void)hipMemcpyAsync(w.plane[0], raw, bytes, hipMemcpyDeviceToDevice, s);
        else (void)hipMemcpyAsync(raw, w.plane[0], bytes, hipMemcpyDeviceToDevice, s);
    }
}

void launch_repack(const DevWeight &w, const uint8_t *raw, hipStream_t s) { repack_common<true>(w, (uint8_t *)raw, s); }
void launch_unpack(const DevWeight &w, uint8_t *raw, hipStream_t s) { repack_common<false>(w, raw, s); }

// ------------------------------------------------------------- dequantize

template <int KIND>
__global__ void k_dequant(WView w, size_t row0, size_t n_rows, size_t cols, float *out) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_rows * cols) return;
    size_t r = i / cols, c = i % cols;
    out[i] = dequant_elem<KIND>(w, row0 + r, c);
}

void launch_dequant(const DevWeight &w, size_t row0, size_t n_rows, float *out, hipStream_t s) {
    size_t n = n_rows * w.cols;
    unsigned grid = (unsigned)((n + 255) / 256);
    WView v = view_of(w);
#define F(K) k_dequant<K><<<grid, 256, 0, s>>>(v, row0, n_rows, w.cols, out)
    AOTK_KIND_SWITCH(w.kind, F)
#undef F
}

// ----------------------------------------------- reference weight encoders

// Source of the values to encode: a device array, or the synthetic generator.
struct Src {
    const float *x;  // null -> synthetic
    size_t cols;
    uint64_t seed;
    uint32_t tensor_index;
    int norm;
    __device__ __forceinline__ float operator()(size_t r, size_t c) const {
        if (x) return x[r * cols + c];
        float v = synth_value(seed, tensor_index, (uint64_t)r * cols + c);
        return norm ? 1.0f + v : v;
    }
};

__device__ __forceinline__ void put16(uint8_t *p, uint16_t v) {
    p[0] = (uint8_t)v;
    p[1] = (uint8_t)(v >> 8);
}

// One thread per block (whole block in one thread, in the reference's order).
template <int KIND>
__global__ void k_encode(Src src, size_t rows, size_t cols, uint8_t *raw) {
    constexpr int BS = (KIND == AOTK_Q4_K || KIND == AOTK_Q5_K || KIND == AOTK_Q6_K) ? 256 : (KIND >= AOTK_Q4_0 ? 32 : 1);
    size_t nb = cols / BS;
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * nb) return;
    size_t r = i / nb, b = i % nb;
    size_t c0 = b * BS;
    size_t rb = row_bytes(KIND, cols);
    if (KIND == AOTK_F32) {
        ((float *)(raw + r * rb))[b] = src(r, c0);
        return;
    }
    if (KIND == AOTK_F16 || KIND == AOTK_BF16) {
        float v = src(r, c0);
        ((uint16_t *)(raw + r * rb))[b] = KIND == AOTK_F16 ? f32_to_f16(v) : f32_to_bf16(v);
        return;
    }
    if (KIND == AOTK_Q4_0 || KIND == AOTK_Q5_0) {
        // quantize.rs:16-71
        uint8_t *o = raw + r * rb + b * (KIND == AOTK_Q4_0 ? 18 : 22);
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < 32; j++) {
            float v = src(r, c0 + j);
            if (fabsf(v) > amax) { amax = fabsf(v); max = v; }
        }
        const float lim = KIND == AOTK_Q4_0 ? -8.0f : -16.0f;
        const int off = KIND == AOTK_Q4_0 ? 8 : 16, top = KIND == AOTK_Q4_0 ? 15 : 31;
        float d = max / lim;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        put16(o, f32_to_f16(d));
        uint32_t qh = 0;
        uint8_t *qs = o + (KIND == AOTK_Q4_0 ? 2 : 6);
        for (int j = 0; j < 16; j++) {
            uint32_t lo = (uint32_t)clampi(round_i(src(r, c0 + j) * id) + off, 0, top);
            uint32_t hi = (uint32_t)clampi(round_i(src(r, c0 + j + 16) * id) + off, 0, top);
            qs[j] = (uint8_t)((lo & 0xF) | ((hi & 0xF) << 4));
            qh |= (lo >> 4) << j;
            qh |= (hi >> 4) << (j + 16);
        }
        if (KIND == AOTK_Q5_0) {
            o[2] = (uint8_t)qh; o[3] = (uint8_t)(qh >> 8); o[4] = (uint8_t)(qh >> 16); o[5] = (uint8_t)(qh >> 24);
        }
        return;
    }
    if (KIND == AOTK_Q8_0) {
        // quantize.rs:74-87
        uint8_t *o = raw + r * rb + b * 34;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(src(r, c0 + j)));
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        put16(o, f32_to_f16(d));
        for (int j = 0; j < 32; j++) o[2 + j] = (uint8_t)(int8_t)clampi(round_i(src(r, c0 + j) * id), -127, 127);
        return;
    }
    if (KIND == AOTK_Q4_K || KIND == AOTK_Q5_K) {
        // quantize.rs:91-204
        constexpr float qmax = KIND == AOTK_Q4_K ? 15.0f : 31.0f;
        uint8_t *o = raw + r * rb + b * (KIND == AOTK_Q4_K ? 144 : 176);
        float sc[8], mn[8];
        for (int j = 0; j < 8; j++) {
            float lo = 3.40282347e38f, hi = -3.40282347e38f;
            for (int l = 0; l < 32; l++) {
                float v = src(r, c0 + 32 * j + l);
                lo = fminf(lo, v);
                hi = fmaxf(hi, v);
            }
            float mnv = fmaxf(-lo, 0.0f);
            float scale = (hi + mnv) / qmax;
            sc[j] = fmaxf(scale, 0.0f);
            mn[j] = mnv;
        }
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; j++) { max_scale = fmaxf(max_scale, sc[j]); max_min = fmaxf(max_min, mn[j]); }
        float d = max_scale / 63.0f, dmin = max_min / 63.0f;
        float inv_d = d != 0.0f ? 1.0f / d : 0.0f;
        float inv_m = dmin != 0.0f ? 1.0f / dmin : 0.0f;
        uint8_t ls[8], lm[8];
        for (int j = 0; j < 8; j++) {
            ls[j] = (uint8_t)clampi(round_i(sc[j] * inv_d), 0, 63);
            lm[j] = (uint8_t)clampi(round_i(mn[j] * inv_m), 0, 63);
        }
        uint16_t dh = f32_to_f16(d), mh = f32_to_f16(dmin);
        d = f16_to_f32(dh);
        dmin = f16_to_f32(mh);
        // f32_to_f16 of an already-rounded half value is the identity.
        put16(o, f32_to_f16(d));
        put16(o + 2, f32_to_f16(dmin));
        uint8_t s12[12];
        for (int j = 0; j < 12; j++) s12[j] = 0;
        for (int j = 0; j < 8; j++) {
            if (j < 4) {
                s12[j] = ls[j];
                s12[j + 4] = lm[j];
            } else {
                s12[j + 4] = (uint8_t)((ls[j] & 0xF) | ((lm[j] & 0xF) << 4));
                s12[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
                s12[j] |= (uint8_t)((lm[j] >> 4) << 6);
            }
        }
        for (int j = 0; j < 12; j++) o[4 + j] = s12[j];
        float inv[8], mm[8];
        for (int j = 0; j < 8; j++) {
            float s = d * (float)ls[j];
            mm[j] = dmin * (float)lm[j];
            inv[j] = s != 0.0f ? 1.0f / s : 0.0f;
        }
        const int qtop = (int)qmax;
        uint32_t qh[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int j = 0; j < 4; j++) {
            for (int l = 0; l < 32; l++) {
                int a = clampi(round_i((src(r, c0 + 64 * j + l) + mm[2 * j]) * inv[2 * j]), 0, qtop);
                int bb = clampi(round_i((src(r, c0 + 64 * j + 32 + l) + mm[2 * j + 1]) * inv[2 * j + 1]), 0, qtop);
                if (KIND == AOTK_Q4_K) {
                    o[16 + 32 * j + l] = (uint8_t)(a | (bb << 4));
                } else {
                    o[48 + 32 * j + l] = (uint8_t)((a & 0xF) | ((bb & 0xF) << 4));
                    uint32_t bits = ((a & 16) ? (1u << (2 * j)) : 0u) | ((bb & 16) ? (2u << (2 * j)) : 0u);
                    qh[l / 4] |= bits << (8 * (l % 4));
                }
            }
        }
        if (KIND == AOTK_Q5_K)
            for (int l = 0; l < 32; l++) o[16 + l] = (uint8_t)(qh[l / 4] >> (8 * (l % 4)));
        return;
    }
    if (KIND == AOTK_Q6_K) {
        // quantize.rs:207-267
        uint8_t *o = raw + r * rb + b * 210;
        float scales[16];
        for (int j = 0; j < 16; j++) {
            float amax = 0.0f, max = 0.0f;
            for (int l = 0; l < 16; l++) {
                float v = src(r, c0 + 16 * j + l);
                if (fabsf(v) > amax) { amax = fabsf(v); max = v; }
            }
            scales[j] = max / -32.0f;
        }
        float max_scale = 0.0f, max_abs = 0.0f;
        for (int j = 0; j < 16; j++)
            if (fabsf(scales[j]) > max_abs) { max_abs = fabsf(scales[j]); max_scale = scales[j]; }
        float iscale = max_scale != 0.0f ? -128.0f / max_scale : 0.0f;
        float d = f16_to_f32(f32_to_f16(1.0f / iscale));
        int8_t ls[16];
        float inv[16];
        for (int j = 0; j < 16; j++) {
            ls[j] = (int8_t)clampi(round_i(iscale * scales[j]), -128, 127);
            float s = d * (float)ls[j];
            inv[j] = s != 0.0f ? 1.0f / s : 0.0f;
        }
        for (int n = 0; n < 2; n++) {
            for (int l = 0; l < 32; l++) {
                int qv[4];
                for (int k = 0; k < 4; k++) {
                    int e = 128 * n + l + 32 * k;
                    qv[k] = clampi(round_i(src(r, c0 + e) * inv[e / 16]), -32, 31) + 32;
                }
                o[64 * n + l] = (uint8_t)((qv[0] & 0xF) | ((qv[2] & 0xF) << 4));
                o[64 * n + l + 32] = (uint8_t)((qv[1] & 0xF) | ((qv[3] & 0xF) << 4));
                o[128 + 32 * n + l] = (uint8_t)((qv[0] >> 4) | ((qv[1] >> 4) << 2) | ((qv[2] >> 4) << 4) | ((qv[3] >> 4) << 6));
            }
        }
        for (int j = 0; j < 16; j++) o[192 + j] = (uint8_t)ls[j];
        put16(o + 208, f32_to_f16(d));
        return;
    }
}

static void encode_any(int kind, Src src, size_t rows, size_t cols, uint8_t *raw, hipStream_t s) {
    size_t n = rows * (cols / block_size(kind));
    unsigned threads = 128;
    unsigned grid = (unsigned)((n + threads - 1) / threads);
#define F(K) k_encode<K><<<grid, threads, 0, s>>>(src, rows, cols, raw)
    AOTK_KIND_SWITCH(kind, F)
#undef F
}

void launch_encode(int kind, const float *x, size_t rows, size_t cols, uint8_t *raw, hipStream_t s) {
    Src src{x, cols, 0, 0, 0};
    encode_any(kind, src, rows, cols, raw, s);
}

void launch_synth(int kind, size_t rows, size_t cols, uint64_t seed, uint32_t tensor_index, int norm, uint8_t *raw,
                  float *scratch, size_t scratch_rows, hipStream_t s) {
    (void)scratch;
    (void)scratch_rows;
    Src src{nullptr, cols, seed, tensor_index, norm};
    encode_any(kind, src, rows, cols, raw, s);
}

// ---------------------------------------------------- activation quantizers

// quantize_q8_k (quant.rs:248-283): one wave per 256-block, 4 values/lane.
// The signed extreme is the first element of largest magnitude.
__global__ void k_quant_q8k(const float *__restrict__ x, size_t nblk, ActQ8K out) {
    size_t blk = (size_t)blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
    int lane = threadIdx.x & 63;
    if (blk >= nblk) return;
    float4 v = ((const float4 *)(x + blk * 256))[lane];
    float vals[4] = {v.x, v.y, v.z, v.w};
    float amax = 0.0f;
    int idx = 0x7fffffff;
    for (int k = 0; k < 4; k++) {
        float a = fabsf(vals[k]);
        if (a > amax) { amax = a; idx = lane * 4 + k; }
    }
    for (int m = 1; m < 64; m <<= 1) {
        float oa = shfl_xor(amax, m);
        int oi = shfl_xor(idx, m);
        if (oa > amax || (oa == amax && oi < idx)) { amax = oa; idx = oi; }
    }
    int8_t *qs = out.qs + blk * 256;
    uint32_t *qt = out.qt ? (uint32_t *)(out.qt + q8k_tiled_off(blk / out.nbt, (int)(blk % out.nbt), out.nbt, 4 * lane)) : nullptr;
    if (amax == 0.0f) {
        ((uint32_t *)qs)[lane] = 0;
        if (qt) *qt = 0;
        if ((lane & 3) == 0) out.bsums[blk * 16 + lane / 4] = 0;
        if (lane == 0) out.d[blk] = 0.0f;
        return;
    }
    float max = x[blk * 256 + idx];
    float iscale = -127.0f / max;
    int q[4];
    int sum = 0;
    for (int k = 0; k < 4; k++) {
        int t = round_i(iscale * vals[k]);
        q[k] = t > 127 ? 127 : t;
        sum += (int8_t)q[k];
    }
    const uint32_t packed = (uint32_t)(q[0] & 0xFF) | ((uint32_t)(q[1] & 0xFF) << 8) | ((uint32_t)(q[2] & 0xFF) << 16) |
                            ((uint32_t)(q[3] & 0xFF) << 24);
    ((uint32_t *)qs)[lane] = packed;
    if (qt) *qt = packed;
    sum += shfl_xor(sum, 1);
    sum += shfl_xor(sum, 2);
    if ((lane & 3) == 0) out.bsums[blk * 16 + lane / 4] = (int16_t)sum;
    if (lane == 0) out.d[blk] = 1.0f / iscale;
}

// quantize_q8_0 (quant.rs:231-245): 32 lanes per block, one value per lane.
__global__ void k_quant_q8_0(const float *__restrict__ x, size_t nblk, ActQ8_0 out) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t blk = i / 32;
    if (blk >= nblk) return;
    float v = x[i];
    // fold(0, max) of |v| (quant.rs:237): NaN never wins, an all-NaN block gives 0
    float amax = fmaxf(0.0f, fabsf(v));
    for (int m = 1; m < 32; m <<= 1) amax = fmaxf(amax, shfl_xor(amax, m));
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    const int q = clampi(round_i(v * id), -127, 127);
    out.qs[i] = (int8_t)q;
    if (out.xh) out.xh[i] = __builtin_bit_cast(uint16_t, (_Float16)q);
    if ((i & 31) == 0) out.d[blk] = d;
}

void launch_quant_q8k(const float *x, size_t n, size_t rows, ActQ8K out, hipStream_t s) {
    size_t nblk = rows * n / 256;
    out.nbt = (int)(n / 256);
    if (rows < 2) out.qt = nullptr;
    k_quant_q8k<<<(unsigned)((nblk + 3) / 4), 256, 0, s>>>(x, nblk, out);
}

void launch_quant_q8_0(const float *x, size_t n, size_t rows, ActQ8_0 out, hipStream_t s) {
    size_t total = rows * n;
    if (rows < 2) out.xh = nullptr;
    k_quant_q8_0<<<(unsigned)((total + 255) / 256), 256, 0, s>>>(x, total / 32, out);
}

// Conversions between the plane layout and the reference's block structs.
__global__ void k_q8k_to_ref(ActQ8K a, size_t nblk, aotk_block_q8_k *out) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk * 256) return;
    size_t b = i / 256;
    int e = (int)(i % 256);
    out[b].qs[e] = a.qs[i];
    if (e < 16) out[b].bsums[e] = a.bsums[b * 16 + e];
    if (e == 0) out[b].d = a.d[b];
}
__global__ void k_ref_to_q8k(const aotk_block_q8_k *in, size_t nblk, ActQ8K a) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk * 256) return;
    size_t b = i / 256;
    int e = (int)(i % 256);
    a.qs[i] = in[b].qs[e];
    if (a.qt) a.qt[q8k_tiled_off(b / a.nbt, (int)(b % a.nbt), a.nbt, e)] = in[b].qs[e];
    if (e < 16) a.bsums[b * 16 + e] = in[b].bsums[e];
    if (e == 0) a.d[b] = in[b].d;
}
__global__ void k_q8_0_to_ref(ActQ8_0 a, size_t nblk, aotk_block_q8_0 *out) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk * 32) return;
    size_t b = i / 32;
    int e = (int)(i % 32);
    out[b].qs[e] = a.qs[i];
    if (e == 0) out[b].d = a.d[b];
}
__global__ void k_ref_to_q8_0(const aotk_block_q8_0 *in, size_t nblk, ActQ8_0 a) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk * 32) return;
    size_t b = i / 32;
    int e = (int)(i % 32);
    a.qs[i] = in[b].qs[e];
    if (a.xh) a.xh[i] = __builtin_bit_cast(uint16_t, (_Float16)in[b].qs[e]);
    if (e == 0) a.d[b] = in[b].d;
}

void launch_q8k_to_ref(ActQ8K a, size_t n, aotk_block_q8_k *out, hipStream_t s) {
    size_t nblk = n / 256;
    k_q8k_to_ref<<<(unsigned)((nblk * 256 + 255) / 256), 256, 0, s>>>(a, nblk, out);
}
void launch_ref_to_q8k(const aotk_block_q8_k *in, size_t n, size_t rows, ActQ8K a, hipStream_t s) {
    size_t nblk = rows * n / 256;
    a.nbt = (int)(n / 256);
    if (rows < 2) a.qt = nullptr;
    k_ref_to_q8k<<<(unsigned)((nblk * 256 + 255) / 256), 256, 0, s>>>(in, nblk, a);
}
void launch_q8_0_to_ref(ActQ8_0 a, size_t n, aotk_block_q8_0 *out, hipStream_t s) {
    size_t nblk = n / 32;
    k_q8_0_to_ref<<<(unsigned)((nblk * 32 + 255) / 256), 256, 0, s>>>(a, nblk, out);
}
void launch_ref_to_q8_0(const aotk_block_q8_0 *in, size_t n, size_t rows, ActQ8_0 a, hipStream_t s) {
    size_t nblk = rows * n / 32;
    k_ref_to_q8_0<<<(unsigned)((nblk * 32 + 255) / 256), 256, 0, s>>>(in, nblk, a);
}

}  // namespace aotk
