/*
 * oracle.c - CPU restatement of aot-llm's quantized inference path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker + CPU baseline); see oracle.h for
 * the scope, the pinning of each part and what stays unpinned. Citations are
 * file:line in the reference repository (p10node/aot-llm).
 *
 * Build: oracle/Makefile (gcc -O2 -mavx2 -mfma -mf16c -ffp-contract=off).
 */
#define _GNU_SOURCE
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

#define QK8_0 32
#define QK_K 256

/* ------------------------------------------------------------------------ */
/* Kinds and sizes: quant.rs:20-87                                          */
/* ------------------------------------------------------------------------ */

static size_t block_size(int kind) {
    switch (kind) {
    case AOTK_F32: case AOTK_F16: case AOTK_BF16: return 1;
    case AOTK_Q4_0: case AOTK_Q5_0: case AOTK_Q8_0: return QK8_0;
    default: return QK_K;
    }
}

static size_t type_size(int kind) {
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

size_t or_row_bytes(int kind, size_t cols) { return cols / block_size(kind) * type_size(kind); }

/* model.rs:85-91 `Kind::activation`: 0 = f32, 1 = Q8_0, 2 = Q8_K */
static int activation(int kind) {
    switch (kind) {
    case AOTK_Q4_0: case AOTK_Q5_0: case AOTK_Q8_0: return 1;
    case AOTK_Q4_K: case AOTK_Q5_K: case AOTK_Q6_K: return 2;
    default: return 0;
    }
}

/* ------------------------------------------------------------------------ */
/* Half precision: quant.rs:96-177                                          */
/* ------------------------------------------------------------------------ */

static inline float bits_f32(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)(h & 0x8000)) << 16;
    uint32_t exp = (h >> 10) & 0x1F;
    uint32_t mant = h & 0x3FF;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            int32_t e = 113;
            uint32_t m = mant;
            while ((m & 0x400) == 0) { m <<= 1; e -= 1; }
            bits = sign | ((uint32_t)e << 23) | ((m & 0x3FF) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (mant << 13);
    }
    return bits_f32(bits);
}

uint16_t or_f32_to_f16(float f) {
    uint32_t x = f32_bits(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000);
    int32_t exp = (int32_t)((x >> 23) & 0xFF);
    uint32_t mant = x & 0x7FFFFF;
    if (exp == 0xFF) return sign | 0x7C00 | (mant != 0 ? 0x200 : 0);
    exp -= 127;
    if (exp > 15) return sign | 0x7C00;
    if (exp < -25) return sign;
    if (exp < -14) {
        uint32_t m = mant | 0x800000;
        uint32_t shift = (uint32_t)(-14 - exp) + 13;
        uint32_t half = 1u << (shift - 1);
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t r = m >> shift;
        if (rem > half || (rem == half && (r & 1) == 1)) r += 1;
        return sign | (uint16_t)r;
    }
    uint32_t r = ((uint32_t)(exp + 15) << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1FFF;
    if (rem > 0x1000 || (rem == 0x1000 && (r & 1) == 1)) r += 1;
    return sign | (uint16_t)r;
}

float or_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

uint16_t or_f32_to_bf16(float f) {
    uint32_t x = f32_bits(f);
    if ((x & 0x7F800000u) == 0x7F800000u) return (uint16_t)((x >> 16) | ((x & 0x7FFFFF) != 0 ? 0x40 : 0));
    uint32_t lsb = (x >> 16) & 1;
    return (uint16_t)((x + 0x7FFF + lsb) >> 16);
}

static inline float read_f16(const uint8_t *b) { return or_f16_to_f32((uint16_t)(b[0] | (b[1] << 8))); }
static inline float read_f32(const uint8_t *b) { float f; memcpy(&f, b, 4); return f; }

/* Rust `x.round() as i32`: round half away from zero, saturating cast. */
static inline int32_t round_i(float x) {
    float r = roundf(x);
    if (r != r) return 0;
    if (r >= 2147483648.0f) return INT32_MAX;
    if (r < -2147483648.0f) return INT32_MIN;
    return (int32_t)r;
}
static inline int32_t clampi(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* ------------------------------------------------------------------------ */
/* Activation quantizers: quant.rs:231-283                                  */
/* ------------------------------------------------------------------------ */

void or_quantize_q8_0(const float *x, size_t n, aotk_block_q8_0 *out) {
    size_t nb = n / QK8_0;
    for (size_t i = 0; i < nb; i++) {
        const float *src = x + i * QK8_0;
        float amax = 0.0f;
        for (int j = 0; j < QK8_0; j++) amax = fmaxf(amax, fabsf(src[j]));
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        out[i].d = d;
        for (int j = 0; j < QK8_0; j++) out[i].qs[j] = (int8_t)clampi(round_i(src[j] * id), -127, 127);
    }
}

void or_quantize_q8_k(const float *x, size_t n, aotk_block_q8_k *out) {
    size_t nb = n / QK_K;
    for (size_t i = 0; i < nb; i++) {
        const float *src = x + i * QK_K;
        aotk_block_q8_k *blk = &out[i];
        float amax = 0.0f, max = 0.0f;
        for (int j = 0; j < QK_K; j++) {
            float a = fabsf(src[j]);
            if (a > amax) { amax = a; max = src[j]; }
        }
        if (amax == 0.0f) {
            memset(blk, 0, sizeof *blk);
            continue;
        }
        float iscale = -127.0f / max;
        for (int j = 0; j < QK_K; j++) {
            int32_t q = round_i(iscale * src[j]);
            if (q > 127) q = 127;
            blk->qs[j] = (int8_t)q;
        }
        for (int j = 0; j < 16; j++) {
            int32_t s = 0;
            for (int k = 0; k < 16; k++) s += blk->qs[j * 16 + k];
            blk->bsums[j] = (int16_t)s;
        }
        blk->d = 1.0f / iscale;
    }
}

/* ------------------------------------------------------------------------ */
/* Dequantizers: quant.rs:292-443                                           */
/* ------------------------------------------------------------------------ */

static inline void scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

void or_dequant_row(int kind, const uint8_t *row, float *out, size_t n) {
    switch (kind) {
    case AOTK_F32:
        for (size_t i = 0; i < n; i++) out[i] = read_f32(row + 4 * i);
        break;
    case AOTK_F16:
        for (size_t i = 0; i < n; i++) out[i] = read_f16(row + 2 * i);
        break;
    case AOTK_BF16:
        for (size_t i = 0; i < n; i++) out[i] = or_bf16_to_f32((uint16_t)(row[2 * i] | (row[2 * i + 1] << 8)));
        break;
    case AOTK_Q4_0:
        for (size_t i = 0; i < n / 32; i++) {
            const uint8_t *b = row + i * 18;
            float d = read_f16(b);
            float *c = out + 32 * i;
            for (int j = 0; j < 16; j++) {
                uint8_t q = b[2 + j];
                c[j] = (float)((int32_t)(q & 0x0F) - 8) * d;
                c[j + 16] = (float)((int32_t)(q >> 4) - 8) * d;
            }
        }
        break;
    case AOTK_Q5_0:
        for (size_t i = 0; i < n / 32; i++) {
            const uint8_t *b = row + i * 22;
            float d = read_f16(b);
            uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
            float *c = out + 32 * i;
            for (int j = 0; j < 16; j++) {
                uint8_t q = b[6 + j];
                uint32_t lo = (uint32_t)(q & 0x0F) | (((qh >> j) & 1) << 4);
                uint32_t hi = (uint32_t)(q >> 4) | (((qh >> (j + 16)) & 1) << 4);
                c[j] = (float)((int32_t)lo - 16) * d;
                c[j + 16] = (float)((int32_t)hi - 16) * d;
            }
        }
        break;
    case AOTK_Q8_0:
        for (size_t i = 0; i < n / 32; i++) {
            const uint8_t *b = row + i * 34;
            float d = read_f16(b);
            for (int j = 0; j < 32; j++) out[32 * i + j] = (float)(int8_t)b[2 + j] * d;
        }
        break;
    case AOTK_Q4_K:
        for (size_t i = 0; i < n / QK_K; i++) {
            const uint8_t *b = row + i * 144;
            float d = read_f16(b), dmin = read_f16(b + 2);
            const uint8_t *scales = b + 4, *qs = b + 16;
            float *c = out + QK_K * i;
            for (int j = 0; j < 4; j++) {
                uint8_t sc1, m1, sc2, m2;
                scale_min_k4(2 * j, scales, &sc1, &m1);
                scale_min_k4(2 * j + 1, scales, &sc2, &m2);
                float d1 = d * (float)sc1, d2 = d * (float)sc2;
                float mm1 = dmin * (float)m1, mm2 = dmin * (float)m2;
                for (int l = 0; l < 32; l++) {
                    uint8_t q = qs[32 * j + l];
                    c[64 * j + l] = d1 * (float)(q & 0xF) - mm1;
                    c[64 * j + 32 + l] = d2 * (float)(q >> 4) - mm2;
                }
            }
        }
        break;
    case AOTK_Q5_K:
        for (size_t i = 0; i < n / QK_K; i++) {
            const uint8_t *b = row + i * 176;
            float d = read_f16(b), dmin = read_f16(b + 2);
            const uint8_t *scales = b + 4, *qh = b + 16, *qs = b + 48;
            float *c = out + QK_K * i;
            for (int j = 0; j < 4; j++) {
                uint8_t sc1, m1, sc2, m2;
                scale_min_k4(2 * j, scales, &sc1, &m1);
                scale_min_k4(2 * j + 1, scales, &sc2, &m2);
                float d1 = d * (float)sc1, d2 = d * (float)sc2;
                float mm1 = dmin * (float)m1, mm2 = dmin * (float)m2;
                uint8_t u1 = (uint8_t)(1u << (2 * j)), u2 = (uint8_t)(2u << (2 * j));
                for (int l = 0; l < 32; l++) {
                    uint8_t q = qs[32 * j + l];
                    int h1 = (qh[l] & u1) ? 16 : 0, h2 = (qh[l] & u2) ? 16 : 0;
                    c[64 * j + l] = d1 * (float)((q & 0xF) + h1) - mm1;
                    c[64 * j + 32 + l] = d2 * (float)((q >> 4) + h2) - mm2;
                }
            }
        }
        break;
    case AOTK_Q6_K:
        for (size_t i = 0; i < n / QK_K; i++) {
            const uint8_t *b = row + i * 210;
            float d = read_f16(b + 208);
            for (int nn = 0; nn < 2; nn++) {
                const uint8_t *ql = b + 64 * nn, *qh = b + 128 + 32 * nn, *sc = b + 192 + 8 * nn;
                float *y = out + QK_K * i + 128 * nn;
                for (int l = 0; l < 32; l++) {
                    int is = l / 16;
                    int32_t q1 = (int32_t)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
                    int32_t q2 = (int32_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    int32_t q3 = (int32_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    int32_t q4 = (int32_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    y[l] = d * (float)(int8_t)sc[is] * (float)q1;
                    y[l + 32] = d * (float)(int8_t)sc[is + 2] * (float)q2;
                    y[l + 64] = d * (float)(int8_t)sc[is + 4] * (float)q3;
                    y[l + 96] = d * (float)(int8_t)sc[is + 6] * (float)q4;
                }
            }
        }
        break;
    }
}

/* ------------------------------------------------------------------------ */
/* Reference weight encoders: quantize.rs:16-294                            */
/* ------------------------------------------------------------------------ */

static void put_u16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

static void sub_block_scale_min(const float *sub, float qmax, float *scale_out, float *min_out) {
    /* quantize.rs:91-102 */
    float lo = 3.40282347e38f, hi = -3.40282347e38f;
    for (int i = 0; i < 32; i++) { lo = fminf(lo, sub[i]); hi = fmaxf(hi, sub[i]); }
    float min = fmaxf(-lo, 0.0f);
    float scale = (hi + min) / qmax;
    *scale_out = fmaxf(scale, 0.0f);
    *min_out = min;
}

static void pack_scales_k4(const uint8_t ls[8], const uint8_t lm[8], uint8_t s[12]) {
    /* quantize.rs:105-119 */
    memset(s, 0, 12);
    for (int j = 0; j < 8; j++) {
        if (j < 4) {
            s[j] = ls[j];
            s[j + 4] = lm[j];
        } else {
            s[j + 4] = (uint8_t)((ls[j] & 0xF) | ((lm[j] & 0xF) << 4));
            s[j - 4] |= (uint8_t)((ls[j] >> 4) << 6);
            s[j] |= (uint8_t)((lm[j] >> 4) << 6);
        }
    }
}

static void encode_k4_block(const float *blk, float qmax, float *d_out, float *dmin_out, uint8_t scales[12], uint8_t q[QK_K]) {
    /* quantize.rs:123-154 */
    float sc[8], mn[8];
    for (int j = 0; j < 8; j++) sub_block_scale_min(blk + 32 * j, qmax, &sc[j], &mn[j]);
    float max_scale = 0.0f, max_min = 0.0f;
    for (int j = 0; j < 8; j++) { max_scale = fmaxf(max_scale, sc[j]); max_min = fmaxf(max_min, mn[j]); }
    float d = max_scale / 63.0f;
    float dmin = max_min / 63.0f;
    float inv_d = d != 0.0f ? 1.0f / d : 0.0f;
    float inv_m = dmin != 0.0f ? 1.0f / dmin : 0.0f;
    uint8_t ls[8], lm[8];
    for (int j = 0; j < 8; j++) {
        ls[j] = (uint8_t)clampi(round_i(sc[j] * inv_d), 0, 63);
        lm[j] = (uint8_t)clampi(round_i(mn[j] * inv_m), 0, 63);
    }
    d = or_f16_to_f32(or_f32_to_f16(d));
    dmin = or_f16_to_f32(or_f32_to_f16(dmin));
    for (int j = 0; j < 8; j++) {
        float s = d * (float)ls[j];
        float m = dmin * (float)lm[j];
        float inv = s != 0.0f ? 1.0f / s : 0.0f;
        for (int l = 0; l < 32; l++) q[32 * j + l] = (uint8_t)clampi(round_i((blk[32 * j + l] + m) * inv), 0, (int32_t)qmax);
    }
    pack_scales_k4(ls, lm, scales);
    *d_out = d;
    *dmin_out = dmin;
}

size_t or_quantize_row(int kind, const float *x, size_t n, uint8_t *out) {
    uint8_t *o = out;
    switch (kind) {
    case AOTK_F32:
        memcpy(o, x, 4 * n);
        return 4 * n;
    case AOTK_F16:
        for (size_t i = 0; i < n; i++) put_u16(o + 2 * i, or_f32_to_f16(x[i]));
        return 2 * n;
    case AOTK_BF16:
        for (size_t i = 0; i < n; i++) put_u16(o + 2 * i, or_f32_to_bf16(x[i]));
        return 2 * n;
    case AOTK_Q4_0: /* quantize.rs:16-40 */
        for (size_t b = 0; b < n / 32; b++, o += 18) {
            const float *blk = x + 32 * b;
            float amax = 0.0f, max = 0.0f;
            for (int j = 0; j < 32; j++) if (fabsf(blk[j]) > amax) { amax = fabsf(blk[j]); max = blk[j]; }
            float d = max / -8.0f;
            float id = d != 0.0f ? 1.0f / d : 0.0f;
            put_u16(o, or_f32_to_f16(d));
            for (int j = 0; j < 16; j++) {
                uint8_t lo = (uint8_t)clampi(round_i(blk[j] * id) + 8, 0, 15);
                uint8_t hi = (uint8_t)clampi(round_i(blk[j + 16] * id) + 8, 0, 15);
                o[2 + j] = (uint8_t)(lo | (hi << 4));
            }
        }
        return (size_t)(o - out);
    case AOTK_Q5_0: /* quantize.rs:43-71 */
        for (size_t b = 0; b < n / 32; b++, o += 22) {
            const float *blk = x + 32 * b;
            float amax = 0.0f, max = 0.0f;
            for (int j = 0; j < 32; j++) if (fabsf(blk[j]) > amax) { amax = fabsf(blk[j]); max = blk[j]; }
            float d = max / -16.0f;
            float id = d != 0.0f ? 1.0f / d : 0.0f;
            uint32_t qh = 0;
            uint8_t qs[16];
            for (int j = 0; j < 16; j++) {
                uint32_t lo = (uint32_t)clampi(round_i(blk[j] * id) + 16, 0, 31);
                uint32_t hi = (uint32_t)clampi(round_i(blk[j + 16] * id) + 16, 0, 31);
                qs[j] = (uint8_t)((lo & 0xF) | ((hi & 0xF) << 4));
                qh |= (lo >> 4) << j;
                qh |= (hi >> 4) << (j + 16);
            }
            put_u16(o, or_f32_to_f16(d));
            o[2] = (uint8_t)qh; o[3] = (uint8_t)(qh >> 8); o[4] = (uint8_t)(qh >> 16); o[5] = (uint8_t)(qh >> 24);
            memcpy(o + 6, qs, 16);
        }
        return (size_t)(o - out);
    case AOTK_Q8_0: /* quantize.rs:74-87 */
        for (size_t b = 0; b < n / 32; b++, o += 34) {
            const float *blk = x + 32 * b;
            float amax = 0.0f;
            for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(blk[j]));
            float d = amax / 127.0f;
            float id = d != 0.0f ? 1.0f / d : 0.0f;
            put_u16(o, or_f32_to_f16(d));
            for (int j = 0; j < 32; j++) o[2 + j] = (uint8_t)(int8_t)clampi(round_i(blk[j] * id), -127, 127);
        }
        return (size_t)(o - out);
    case AOTK_Q4_K: /* quantize.rs:157-172 */
        for (size_t b = 0; b < n / QK_K; b++, o += 144) {
            float d, dmin;
            uint8_t scales[12], q[QK_K];
            encode_k4_block(x + QK_K * b, 15.0f, &d, &dmin, scales, q);
            put_u16(o, or_f32_to_f16(d));
            put_u16(o + 2, or_f32_to_f16(dmin));
            memcpy(o + 4, scales, 12);
            for (int j = 0; j < 4; j++)
                for (int l = 0; l < 32; l++) o[16 + 32 * j + l] = (uint8_t)(q[64 * j + l] | (q[64 * j + 32 + l] << 4));
        }
        return (size_t)(o - out);
    case AOTK_Q5_K: /* quantize.rs:175-204 */
        for (size_t b = 0; b < n / QK_K; b++, o += 176) {
            float d, dmin;
            uint8_t scales[12], q[QK_K], qh[32], qs[128];
            encode_k4_block(x + QK_K * b, 31.0f, &d, &dmin, scales, q);
            put_u16(o, or_f32_to_f16(d));
            put_u16(o + 2, or_f32_to_f16(dmin));
            memcpy(o + 4, scales, 12);
            memset(qh, 0, 32);
            for (int j = 0; j < 4; j++) {
                uint8_t u1 = (uint8_t)(1u << (2 * j)), u2 = (uint8_t)(2u << (2 * j));
                for (int l = 0; l < 32; l++) {
                    uint8_t a = q[64 * j + l], bb = q[64 * j + 32 + l];
                    qs[32 * j + l] = (uint8_t)((a & 0xF) | ((bb & 0xF) << 4));
                    if (a & 16) qh[l] |= u1;
                    if (bb & 16) qh[l] |= u2;
                }
            }
            memcpy(o + 16, qh, 32);
            memcpy(o + 48, qs, 128);
        }
        return (size_t)(o - out);
    case AOTK_Q6_K: /* quantize.rs:207-267 */
        for (size_t b = 0; b < n / QK_K; b++, o += 210) {
            const float *blk = x + QK_K * b;
            float scales[16];
            for (int j = 0; j < 16; j++) {
                float amax = 0.0f, max = 0.0f;
                for (int l = 0; l < 16; l++) if (fabsf(blk[16 * j + l]) > amax) { amax = fabsf(blk[16 * j + l]); max = blk[16 * j + l]; }
                scales[j] = max / -32.0f;
            }
            float max_scale = 0.0f, max_abs = 0.0f;
            for (int j = 0; j < 16; j++) if (fabsf(scales[j]) > max_abs) { max_abs = fabsf(scales[j]); max_scale = scales[j]; }
            float iscale = max_scale != 0.0f ? -128.0f / max_scale : 0.0f;
            float d = or_f16_to_f32(or_f32_to_f16(1.0f / iscale));
            int8_t ls[16];
            for (int j = 0; j < 16; j++) ls[j] = (int8_t)clampi(round_i(iscale * scales[j]), -128, 127);
            uint8_t q[QK_K];
            for (int j = 0; j < 16; j++) {
                float s = d * (float)ls[j];
                float inv = s != 0.0f ? 1.0f / s : 0.0f;
                for (int l = 0; l < 16; l++) q[16 * j + l] = (uint8_t)(clampi(round_i(blk[16 * j + l] * inv), -32, 31) + 32);
            }
            uint8_t *ql = o, *qh = o + 128;
            for (int nn = 0; nn < 2; nn++) {
                for (int l = 0; l < 32; l++) {
                    uint8_t q1 = q[128 * nn + l], q2 = q[128 * nn + l + 32], q3 = q[128 * nn + l + 64], q4 = q[128 * nn + l + 96];
                    ql[64 * nn + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
                    ql[64 * nn + l + 32] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
                    qh[32 * nn + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
                }
            }
            for (int j = 0; j < 16; j++) o[192 + j] = (uint8_t)ls[j];
            put_u16(o + 208, or_f32_to_f16(d));
        }
        return (size_t)(o - out);
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Scalar reference dots: matvec.rs:30-192                                  */
/* ------------------------------------------------------------------------ */

float or_dot_scalar(int kind, const uint8_t *w, const void *xv, size_t cols) {
    float sum = 0.0f;
    switch (kind) {
    case AOTK_Q4_0: {
        const aotk_block_q8_0 *x = xv;
        for (size_t i = 0; i < cols / 32; i++) {
            const uint8_t *b = w + i * 18;
            float d = read_f16(b);
            int32_t s = 0;
            for (int j = 0; j < 16; j++) {
                uint8_t q = b[2 + j];
                s += ((int32_t)(q & 0x0F) - 8) * x[i].qs[j];
                s += ((int32_t)(q >> 4) - 8) * x[i].qs[j + 16];
            }
            sum += (float)s * d * x[i].d;
        }
        break;
    }
    case AOTK_Q5_0: {
        const aotk_block_q8_0 *x = xv;
        for (size_t i = 0; i < cols / 32; i++) {
            const uint8_t *b = w + i * 22;
            float d = read_f16(b);
            uint32_t qh = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
            int32_t s = 0;
            for (int j = 0; j < 16; j++) {
                uint8_t q = b[6 + j];
                int32_t lo = (int32_t)((q & 0x0F) | (((qh >> j) & 1) << 4)) - 16;
                int32_t hi = (int32_t)((q >> 4) | (((qh >> (j + 16)) & 1) << 4)) - 16;
                s += lo * x[i].qs[j];
                s += hi * x[i].qs[j + 16];
            }
            sum += (float)s * d * x[i].d;
        }
        break;
    }
    case AOTK_Q8_0: {
        const aotk_block_q8_0 *x = xv;
        for (size_t i = 0; i < cols / 32; i++) {
            const uint8_t *b = w + i * 34;
            float d = read_f16(b);
            int32_t s = 0;
            for (int j = 0; j < 32; j++) s += (int32_t)(int8_t)b[2 + j] * x[i].qs[j];
            sum += (float)s * d * x[i].d;
        }
        break;
    }
    case AOTK_Q4_K: {
        const aotk_block_q8_k *x = xv;
        for (size_t i = 0; i < cols / QK_K; i++) {
            const uint8_t *b = w + i * 144;
            float d = read_f16(b) * x[i].d;
            float dmin = read_f16(b + 2) * x[i].d;
            const uint8_t *scales = b + 4, *qs = b + 16;
            int32_t sumi = 0, summ = 0;
            for (int j = 0; j < 8; j++) {
                uint8_t sc, m;
                scale_min_k4(j, scales, &sc, &m);
                summ += (int32_t)m * ((int32_t)x[i].bsums[2 * j] + x[i].bsums[2 * j + 1]);
                int c = j / 2;
                int32_t s = 0;
                for (int l = 0; l < 32; l++) {
                    uint8_t q = qs[32 * c + l];
                    uint8_t v = (j % 2 == 0) ? (q & 0x0F) : (q >> 4);
                    s += (int32_t)v * x[i].qs[32 * j + l];
                }
                sumi += (int32_t)sc * s;
            }
            sum += d * (float)sumi - dmin * (float)summ;
        }
        break;
    }
    case AOTK_Q5_K: {
        const aotk_block_q8_k *x = xv;
        for (size_t i = 0; i < cols / QK_K; i++) {
            const uint8_t *b = w + i * 176;
            float d = read_f16(b) * x[i].d;
            float dmin = read_f16(b + 2) * x[i].d;
            const uint8_t *scales = b + 4, *qh = b + 16, *qs = b + 48;
            int32_t sumi = 0, summ = 0;
            for (int j = 0; j < 8; j++) {
                uint8_t sc, m;
                scale_min_k4(j, scales, &sc, &m);
                summ += (int32_t)m * ((int32_t)x[i].bsums[2 * j] + x[i].bsums[2 * j + 1]);
                int c = j / 2;
                uint8_t hbit = (uint8_t)(1u << j);
                int32_t s = 0;
                for (int l = 0; l < 32; l++) {
                    uint8_t q = qs[32 * c + l];
                    uint8_t v = (j % 2 == 0) ? (q & 0x0F) : (q >> 4);
                    if (qh[l] & hbit) v += 16;
                    s += (int32_t)v * x[i].qs[32 * j + l];
                }
                sumi += (int32_t)sc * s;
            }
            sum += d * (float)sumi - dmin * (float)summ;
        }
        break;
    }
    case AOTK_Q6_K: {
        const aotk_block_q8_k *x = xv;
        for (size_t i = 0; i < cols / QK_K; i++) {
            const uint8_t *b = w + i * 210;
            float d = read_f16(b + 208) * x[i].d;
            int32_t sumi = 0;
            for (int nn = 0; nn < 2; nn++) {
                const uint8_t *ql = b + 64 * nn, *qh = b + 128 + 32 * nn, *sc = b + 192 + 8 * nn;
                const int8_t *y = x[i].qs + 128 * nn;
                for (int l = 0; l < 32; l++) {
                    int is = l / 16;
                    int32_t q1 = (int32_t)((ql[l] & 0xF) | ((qh[l] & 3) << 4)) - 32;
                    int32_t q2 = (int32_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                    int32_t q3 = (int32_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                    int32_t q4 = (int32_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                    sumi += (int32_t)(int8_t)sc[is] * q1 * y[l];
                    sumi += (int32_t)(int8_t)sc[is + 2] * q2 * y[l + 32];
                    sumi += (int32_t)(int8_t)sc[is + 4] * q3 * y[l + 64];
                    sumi += (int32_t)(int8_t)sc[is + 6] * q4 * y[l + 96];
                }
            }
            sum += d * (float)sumi;
        }
        break;
    }
    case AOTK_F16: {
        const float *x = xv;
        for (size_t i = 0; i < cols; i++) sum += read_f16(w + 2 * i) * x[i];
        break;
    }
    case AOTK_BF16: {
        const float *x = xv;
        for (size_t i = 0; i < cols; i++) sum += or_bf16_to_f32((uint16_t)(w[2 * i] | (w[2 * i + 1] << 8))) * x[i];
        break;
    }
    case AOTK_F32: {
        const float *x = xv;
        for (size_t i = 0; i < cols; i++) sum += read_f32(w + 4 * i) * x[i];
        break;
    }
    }
    return sum;
}

/* ------------------------------------------------------------------------ */
/* AVX2 + FMA + F16C dots: simd_avx2.rs (same intrinsics, same order)       */
/* ------------------------------------------------------------------------ */

static inline int32_t hsum_i32(__m256i v) {
    /* simd_avx2.rs:19-25 */
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4E));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x01));
    return _mm_cvtsi128_si32(s);
}

static inline float hsum_f32(__m256 v) {
    /* simd_avx2.rs:27-34: ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)) */
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 0x55));
    return _mm_cvtss_f32(s);
}

static inline __m256i mul_sum_i8_pairs(__m256i a, __m256i b) {
    /* simd_avx2.rs:39-46 */
    __m256i ax = _mm256_sign_epi8(a, a);
    __m256i sy = _mm256_sign_epi8(b, a);
    __m256i dot = _mm256_maddubs_epi16(ax, sy);
    return _mm256_madd_epi16(dot, _mm256_set1_epi16(1));
}

static inline __m256i nibbles_32(const uint8_t *p) {
    /* simd_avx2.rs:51-55 */
    __m128i tmp = _mm_loadu_si128((const __m128i *)p);
    __m256i both = _mm256_set_m128i(_mm_srli_epi16(tmp, 4), tmp);
    return _mm256_and_si256(both, _mm256_set1_epi8(0x0F));
}

static inline __m256i bytes_from_bits_32(const uint8_t *p) {
    /* simd_avx2.rs:77-84 */
    int32_t qh;
    memcpy(&qh, p, 4);
    __m256i shuf = _mm256_set_epi64x(0x0303030303030303LL, 0x0202020202020202LL, 0x0101010101010101LL, 0);
    __m256i bytes = _mm256_shuffle_epi8(_mm256_set1_epi32(qh), shuf);
    __m256i bit_mask = _mm256_set1_epi64x(0x7fbfdfeff7fbfdfeLL);
    return _mm256_cmpeq_epi8(_mm256_or_si256(bytes, bit_mask), _mm256_set1_epi64x(-1));
}

static inline __m256i q5_0_elems(const uint8_t *b) {
    /* simd_avx2.rs:89-94 */
    __m256i bx = nibbles_32(b + 6);
    __m256i bxhi = _mm256_andnot_si256(bytes_from_bits_32(b + 2), _mm256_set1_epi8((char)0xF0));
    return _mm256_or_si256(bx, bxhi);
}

static inline __m256i q8_0_like_elems(int kind, const uint8_t *b) {
    switch (kind) {
    case AOTK_Q4_0: return _mm256_sub_epi8(nibbles_32(b + 2), _mm256_set1_epi8(8));
    case AOTK_Q5_0: return q5_0_elems(b);
    default: return _mm256_loadu_si256((const __m256i *)(b + 2));
    }
}

static float avx2_q8_0_family(int kind, const uint8_t *w, const aotk_block_q8_0 *x, size_t nb) {
    /* simd_avx2.rs:58-73, :98-112, :115-129 */
    size_t bs = type_size(kind);
    __m256 acc = _mm256_setzero_ps();
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = w + i * bs;
        __m256 d = _mm256_set1_ps(read_f16(b) * x[i].d);
        __m256i bx = q8_0_like_elems(kind, b);
        __m256i by = _mm256_loadu_si256((const __m256i *)x[i].qs);
        __m256 p = _mm256_cvtepi32_ps(mul_sum_i8_pairs(bx, by));
        acc = _mm256_fmadd_ps(d, p, acc);
    }
    return hsum_f32(acc);
}

static void k4_scales(const uint8_t *scales, const aotk_block_q8_k *y, int16_t sc[8], int32_t *summ) {
    /* simd_avx2.rs:133-143 */
    int32_t s = 0;
    for (int j = 0; j < 8; j++) {
        uint8_t a, m;
        scale_min_k4(j, scales, &a, &m);
        sc[j] = a;
        s += (int32_t)m * ((int32_t)y->bsums[2 * j] + y->bsums[2 * j + 1]);
    }
    *summ = s;
}

static float avx2_q4_k(const uint8_t *w, const aotk_block_q8_k *x, size_t nb) {
    /* simd_avx2.rs:146-172 */
    __m256i m4 = _mm256_set1_epi8(0x0F);
    float sumf = 0.0f;
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = w + i * 144;
        float d = read_f16(b) * x[i].d;
        float dmin = read_f16(b + 2) * x[i].d;
        int16_t sc[8];
        int32_t summ;
        k4_scales(b + 4, &x[i], sc, &summ);
        const uint8_t *qs = b + 16;
        const int8_t *yp = x[i].qs;
        __m256i sumi = _mm256_setzero_si256();
        for (int j = 0; j < 4; j++) {
            __m256i q = _mm256_loadu_si256((const __m256i *)(qs + 32 * j));
            __m256i lo = _mm256_and_si256(q, m4);
            __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);
            __m256i y0 = _mm256_loadu_si256((const __m256i *)(yp + 64 * j));
            __m256i y1 = _mm256_loadu_si256((const __m256i *)(yp + 64 * j + 32));
            __m256i p0 = _mm256_madd_epi16(_mm256_maddubs_epi16(lo, y0), _mm256_set1_epi16(sc[2 * j]));
            __m256i p1 = _mm256_madd_epi16(_mm256_maddubs_epi16(hi, y1), _mm256_set1_epi16(sc[2 * j + 1]));
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(p0, p1));
        }
        sumf += d * (float)hsum_i32(sumi) - dmin * (float)summ;
    }
    return sumf;
}

static inline __m256i qh_bit_to_16(__m256i v, int bit) {
    /* simd_avx2.rs:178-193 */
    __m256i m = _mm256_set1_epi8(0x10);
    __m256i s;
    switch (bit) {
    case 0: s = _mm256_slli_epi16(v, 4); break;
    case 1: s = _mm256_slli_epi16(v, 3); break;
    case 2: s = _mm256_slli_epi16(v, 2); break;
    case 3: s = _mm256_slli_epi16(v, 1); break;
    case 4: s = v; break;
    case 5: s = _mm256_srli_epi16(v, 1); break;
    case 6: s = _mm256_srli_epi16(v, 2); break;
    default: s = _mm256_srli_epi16(v, 3); break;
    }
    return _mm256_and_si256(s, m);
}

static float avx2_q5_k(const uint8_t *w, const aotk_block_q8_k *x, size_t nb) {
    /* simd_avx2.rs:195-222 */
    __m256i m4 = _mm256_set1_epi8(0x0F);
    float sumf = 0.0f;
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = w + i * 176;
        float d = read_f16(b) * x[i].d;
        float dmin = read_f16(b + 2) * x[i].d;
        int16_t sc[8];
        int32_t summ;
        k4_scales(b + 4, &x[i], sc, &summ);
        __m256i qh = _mm256_loadu_si256((const __m256i *)(b + 16));
        const uint8_t *qs = b + 48;
        const int8_t *yp = x[i].qs;
        __m256i sumi = _mm256_setzero_si256();
        for (int j = 0; j < 4; j++) {
            __m256i q = _mm256_loadu_si256((const __m256i *)(qs + 32 * j));
            __m256i lo = _mm256_or_si256(_mm256_and_si256(q, m4), qh_bit_to_16(qh, 2 * j));
            __m256i hi = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(q, 4), m4), qh_bit_to_16(qh, 2 * j + 1));
            __m256i y0 = _mm256_loadu_si256((const __m256i *)(yp + 64 * j));
            __m256i y1 = _mm256_loadu_si256((const __m256i *)(yp + 64 * j + 32));
            __m256i p0 = _mm256_madd_epi16(_mm256_maddubs_epi16(lo, y0), _mm256_set1_epi16(sc[2 * j]));
            __m256i p1 = _mm256_madd_epi16(_mm256_maddubs_epi16(hi, y1), _mm256_set1_epi16(sc[2 * j + 1]));
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(p0, p1));
        }
        sumf += d * (float)hsum_i32(sumi) - dmin * (float)summ;
    }
    return sumf;
}

static inline void q6_k_quarters(const uint8_t *b, int n, __m256i qv[4]) {
    /* simd_avx2.rs:243-250 */
    __m256i m4 = _mm256_set1_epi8(0x0F), m30 = _mm256_set1_epi8(0x30);
    const uint8_t *ql = b + 64 * n, *qh = b + 128 + 32 * n;
    __m256i ql0 = _mm256_loadu_si256((const __m256i *)ql);
    __m256i ql32 = _mm256_loadu_si256((const __m256i *)(ql + 32));
    __m256i qhv = _mm256_loadu_si256((const __m256i *)qh);
    qv[0] = _mm256_or_si256(_mm256_and_si256(ql0, m4), _mm256_and_si256(_mm256_slli_epi16(qhv, 4), m30));
    qv[1] = _mm256_or_si256(_mm256_and_si256(ql32, m4), _mm256_and_si256(_mm256_slli_epi16(qhv, 2), m30));
    qv[2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(ql0, 4), m4), _mm256_and_si256(qhv, m30));
    qv[3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(ql32, 4), m4), _mm256_and_si256(_mm256_srli_epi16(qhv, 2), m30));
}

static float avx2_q6_k(const uint8_t *w, const aotk_block_q8_k *x, size_t nb) {
    /* simd_avx2.rs:225-267 */
    float sumf = 0.0f;
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = w + i * 210;
        float d = read_f16(b + 208) * x[i].d;
        const int8_t *scales = (const int8_t *)(b + 192);
        int32_t bias = 0;
        for (int k = 0; k < 16; k++) bias += (int32_t)scales[k] * x[i].bsums[k];
        __m256i sumi = _mm256_setzero_si256();
        for (int n = 0; n < 2; n++) {
            const int8_t *sc = scales + 8 * n;
            const int8_t *yp = x[i].qs + 128 * n;
            __m256i qv[4];
            q6_k_quarters(b, n, qv);
            for (int k = 0; k < 4; k++) {
                __m256i yv = _mm256_loadu_si256((const __m256i *)(yp + 32 * k));
                __m256i p16 = _mm256_maddubs_epi16(qv[k], yv);
                __m256i scv = _mm256_set_m128i(_mm_set1_epi16(sc[2 * k + 1]), _mm_set1_epi16(sc[2 * k]));
                sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(p16, scv));
            }
        }
        sumf += d * (float)(hsum_i32(sumi) - 32 * bias);
    }
    return sumf;
}

static float avx2_f16(const uint8_t *w, const float *x, size_t n) {
    /* simd_avx2.rs:433-452 */
    __m256 acc = _mm256_setzero_ps();
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        __m128i h = _mm_loadu_si128((const __m128i *)(w + 2 * i));
        acc = _mm256_fmadd_ps(_mm256_cvtph_ps(h), _mm256_loadu_ps(x + i), acc);
    }
    float sum = hsum_f32(acc);
    for (; i < n; i++) sum += read_f16(w + 2 * i) * x[i];
    return sum;
}

static float avx2_bf16(const uint8_t *w, const float *x, size_t n) {
    /* simd_avx2.rs:455-474 */
    __m256 acc = _mm256_setzero_ps();
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        __m128i h = _mm_loadu_si128((const __m128i *)(w + 2 * i));
        __m256 f = _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(h), 16));
        acc = _mm256_fmadd_ps(f, _mm256_loadu_ps(x + i), acc);
    }
    float sum = hsum_f32(acc);
    for (; i < n; i++) sum += or_bf16_to_f32((uint16_t)(w[2 * i] | (w[2 * i + 1] << 8))) * x[i];
    return sum;
}

static float avx2_f32(const uint8_t *w, const float *x, size_t n) {
    /* simd_avx2.rs:477-493 */
    __m256 acc = _mm256_setzero_ps();
    size_t i = 0;
    for (; i + 8 <= n; i += 8) acc = _mm256_fmadd_ps(_mm256_loadu_ps((const float *)(w + 4 * i)), _mm256_loadu_ps(x + i), acc);
    float sum = hsum_f32(acc);
    for (; i < n; i++) sum += read_f32(w + 4 * i) * x[i];
    return sum;
}

float or_dot_avx2(int kind, const uint8_t *w, const void *x, size_t cols) {
    switch (kind) {
    case AOTK_Q4_0: case AOTK_Q5_0: case AOTK_Q8_0: return avx2_q8_0_family(kind, w, x, cols / 32);
    case AOTK_Q4_K: return avx2_q4_k(w, x, cols / QK_K);
    case AOTK_Q5_K: return avx2_q5_k(w, x, cols / QK_K);
    case AOTK_Q6_K: return avx2_q6_k(w, x, cols / QK_K);
    case AOTK_F16: return avx2_f16(w, x, cols);
    case AOTK_BF16: return avx2_bf16(w, x, cols);
    default: return avx2_f32(w, x, cols);
    }
}

/* 1x4 micro-kernels: simd_avx2.rs:273-430 */
static void avx2_q8_0_family_x4(int kind, const uint8_t *w, const aotk_block_q8_0 *const xs[4], size_t nb, float out[4]) {
    size_t bs = type_size(kind);
    __m256 acc[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = w + i * bs;
        float d = read_f16(b);
        __m256i bx = q8_0_like_elems(kind, b);
        __m256i ax = _mm256_sign_epi8(bx, bx);
        for (int k = 0; k < 4; k++) {
            const aotk_block_q8_0 *y = &xs[k][i];
            __m256i by = _mm256_loadu_si256((const __m256i *)y->qs);
            __m256i sy = _mm256_sign_epi8(by, bx);
            __m256 p = _mm256_cvtepi32_ps(_mm256_madd_epi16(_mm256_maddubs_epi16(ax, sy), _mm256_set1_epi16(1)));
            acc[k] = _mm256_fmadd_ps(_mm256_set1_ps(d * y->d), p, acc[k]);
        }
    }
    for (int k = 0; k < 4; k++) out[k] = hsum_f32(acc[k]);
}

static void avx2_q4_k_x4(const uint8_t *w, const aotk_block_q8_k *const xs[4], size_t nb, float out[4]) {
    __m256i m4 = _mm256_set1_epi8(0x0F);
    float sumf[4] = {0, 0, 0, 0};
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = w + i * 144;
        float d = read_f16(b), dmin = read_f16(b + 2);
        int16_t sc[8];
        int32_t mn[8];
        for (int j = 0; j < 8; j++) {
            uint8_t a, m;
            scale_min_k4(j, b + 4, &a, &m);
            sc[j] = a;
            mn[j] = m;
        }
        const uint8_t *qs = b + 16;
        __m256i sumi[4] = {_mm256_setzero_si256(), _mm256_setzero_si256(), _mm256_setzero_si256(), _mm256_setzero_si256()};
        for (int j = 0; j < 4; j++) {
            __m256i q = _mm256_loadu_si256((const __m256i *)(qs + 32 * j));
            __m256i lo = _mm256_and_si256(q, m4);
            __m256i hi = _mm256_and_si256(_mm256_srli_epi16(q, 4), m4);
            __m256i s0 = _mm256_set1_epi16(sc[2 * j]), s1 = _mm256_set1_epi16(sc[2 * j + 1]);
            for (int k = 0; k < 4; k++) {
                const int8_t *yp = xs[k][i].qs;
                __m256i y0 = _mm256_loadu_si256((const __m256i *)(yp + 64 * j));
                __m256i y1 = _mm256_loadu_si256((const __m256i *)(yp + 64 * j + 32));
                __m256i p0 = _mm256_madd_epi16(_mm256_maddubs_epi16(lo, y0), s0);
                __m256i p1 = _mm256_madd_epi16(_mm256_maddubs_epi16(hi, y1), s1);
                sumi[k] = _mm256_add_epi32(sumi[k], _mm256_add_epi32(p0, p1));
            }
        }
        for (int k = 0; k < 4; k++) {
            const aotk_block_q8_k *y = &xs[k][i];
            int32_t summ = 0;
            for (int j = 0; j < 8; j++) summ += mn[j] * ((int32_t)y->bsums[2 * j] + y->bsums[2 * j + 1]);
            sumf[k] += (d * y->d) * (float)hsum_i32(sumi[k]) - (dmin * y->d) * (float)summ;
        }
    }
    for (int k = 0; k < 4; k++) out[k] = sumf[k];
}

static void avx2_q6_k_x4(const uint8_t *w, const aotk_block_q8_k *const xs[4], size_t nb, float out[4]) {
    float sumf[4] = {0, 0, 0, 0};
    for (size_t i = 0; i < nb; i++) {
        const uint8_t *b = w + i * 210;
        float d = read_f16(b + 208);
        const int8_t *scales = (const int8_t *)(b + 192);
        __m256i sumi[4] = {_mm256_setzero_si256(), _mm256_setzero_si256(), _mm256_setzero_si256(), _mm256_setzero_si256()};
        for (int n = 0; n < 2; n++) {
            const int8_t *sc = scales + 8 * n;
            __m256i qv[4];
            q6_k_quarters(b, n, qv);
            for (int kq = 0; kq < 4; kq++) {
                __m256i scv = _mm256_set_m128i(_mm_set1_epi16(sc[2 * kq + 1]), _mm_set1_epi16(sc[2 * kq]));
                for (int k = 0; k < 4; k++) {
                    const int8_t *yp = xs[k][i].qs + 128 * n;
                    __m256i yv = _mm256_loadu_si256((const __m256i *)(yp + 32 * kq));
                    sumi[k] = _mm256_add_epi32(sumi[k], _mm256_madd_epi16(_mm256_maddubs_epi16(qv[kq], yv), scv));
                }
            }
        }
        for (int k = 0; k < 4; k++) {
            const aotk_block_q8_k *y = &xs[k][i];
            int32_t bias = 0;
            for (int j = 0; j < 16; j++) bias += (int32_t)scales[j] * y->bsums[j];
            sumf[k] += (d * y->d) * (float)(hsum_i32(sumi[k]) - 32 * bias);
        }
    }
    for (int k = 0; k < 4; k++) out[k] = sumf[k];
}

int or_dot_avx2_x4(int kind, const uint8_t *w, const void *const xs[4], size_t cols, float out[4]) {
    switch (kind) {
    case AOTK_Q4_0: case AOTK_Q5_0: case AOTK_Q8_0:
        avx2_q8_0_family_x4(kind, w, (const aotk_block_q8_0 *const *)xs, cols / 32, out);
        return 0;
    case AOTK_Q4_K:
        avx2_q4_k_x4(w, (const aotk_block_q8_k *const *)xs, cols / QK_K, out);
        return 0;
    case AOTK_Q6_K:
        avx2_q6_k_x4(w, (const aotk_block_q8_k *const *)xs, cols / QK_K, out);
        return 0;
    default:
        return -1;
    }
}

/* ------------------------------------------------------------------------ */
/* Fork-join pool: pool.rs:66-159                                           */
/* ------------------------------------------------------------------------ */

typedef void (*job_fn)(void *ctx, int tid, int nth);

struct or_pool {
    int n;
    pthread_t *threads;
    _Atomic unsigned long epoch;
    _Atomic int pending;
    _Atomic int stop;
    job_fn fn;
    void *ctx;
};

typedef struct { or_pool *p; int tid; } worker_arg;

static void *worker_main(void *arg) {
    worker_arg *wa = arg;
    or_pool *p = wa->p;
    int tid = wa->tid;
    free(wa);
    unsigned long seen = 0;
    for (;;) {
        unsigned spins = 0;
        for (;;) {
            unsigned long e = atomic_load_explicit(&p->epoch, memory_order_acquire);
            if (e != seen) { seen = e; break; }
            if (atomic_load_explicit(&p->stop, memory_order_relaxed)) return NULL;
            spins++;
            if (spins < 50000) __builtin_ia32_pause();
            else if (spins < 60000) sched_yield();
            else usleep(200);
        }
        p->fn(p->ctx, tid, p->n);
        atomic_fetch_sub_explicit(&p->pending, 1, memory_order_acq_rel);
    }
}

or_pool *or_pool_new(int n_threads) {
    if (n_threads < 1) n_threads = 1;
    or_pool *p = calloc(1, sizeof *p);
    p->n = n_threads;
    p->threads = calloc((size_t)n_threads, sizeof(pthread_t));
    for (int t = 1; t < n_threads; t++) {
        worker_arg *wa = malloc(sizeof *wa);
        wa->p = p;
        wa->tid = t;
        pthread_create(&p->threads[t], NULL, worker_main, wa);
    }
    return p;
}

void or_pool_free(or_pool *p) {
    if (!p) return;
    atomic_store(&p->stop, 1);
    for (int t = 1; t < p->n; t++) pthread_join(p->threads[t], NULL);
    free(p->threads);
    free(p);
}

int or_pool_threads(const or_pool *p) { return p ? p->n : 1; }

static void pool_run(or_pool *p, job_fn fn, void *ctx) {
    if (!p || p->n == 1) { fn(ctx, 0, 1); return; }
    p->fn = fn;
    p->ctx = ctx;
    atomic_store_explicit(&p->pending, p->n - 1, memory_order_relaxed);
    atomic_fetch_add_explicit(&p->epoch, 1, memory_order_release);
    fn(ctx, 0, p->n);
    while (atomic_load_explicit(&p->pending, memory_order_acquire) != 0) __builtin_ia32_pause();
}

typedef void (*range_fn)(void *ctx, size_t start, size_t end);
typedef struct { range_fn fn; void *ctx; size_t n, chunk; _Atomic size_t next; } chunks_job;

static void chunks_worker(void *c, int tid, int nth) {
    (void)tid; (void)nth;
    chunks_job *j = c;
    for (;;) {
        size_t s = atomic_fetch_add_explicit(&j->next, j->chunk, memory_order_relaxed);
        if (s >= j->n) break;
        size_t e = s + j->chunk < j->n ? s + j->chunk : j->n;
        j->fn(j->ctx, s, e);
    }
}

static void pool_run_chunks(or_pool *p, size_t n, size_t chunk, range_fn fn, void *ctx) {
    /* pool.rs:91-108 */
    if (chunk < 1) chunk = 1;
    if (n == 0) return;
    if (!p || p->n == 1 || n <= chunk) { fn(ctx, 0, n); return; }
    chunks_job j = {fn, ctx, n, chunk, 0};
    pool_run(p, chunks_worker, &j);
}

static void split_range(size_t n, int tid, int nth, size_t *s, size_t *e) {
    /* pool.rs:154-159 */
    size_t chunk = (n + (size_t)nth - 1) / (size_t)nth;
    size_t a = (size_t)tid * chunk, b = (size_t)(tid + 1) * chunk;
    *s = a < n ? a : n;
    *e = b < n ? b : n;
}

/* ------------------------------------------------------------------------ */
/* Matvec / matmul drivers: matvec.rs:300-583                               */
/* ------------------------------------------------------------------------ */

static float dot_dispatch(int kernels, int kind, const uint8_t *w, const void *x, size_t cols) {
    return kernels ? or_dot_avx2(kind, w, x, cols) : or_dot_scalar(kind, w, x, cols);
}

typedef struct { int kernels, kind; float *out; const uint8_t *w; const void *x; size_t rb, cols; } mv_ctx;

static void mv_range(void *c, size_t s, size_t e) {
    mv_ctx *m = c;
    for (size_t r = s; r < e; r++) m->out[r] = dot_dispatch(m->kernels, m->kind, m->w + r * m->rb, m->x, m->cols);
}

void or_matvec(or_pool *p, int kernels, int kind, float *out, const uint8_t *w, const void *x, size_t rows, size_t cols) {
    mv_ctx c = {kernels, kind, out, w, x, or_row_bytes(kind, cols), cols};
    size_t nth = (size_t)or_pool_threads(p);
    size_t chunk = rows / (nth * 8);
    if (chunk < 8) chunk = 8; /* matvec.rs:316-318 row_chunk */
    pool_run_chunks(p, rows, chunk, mv_range, &c);
}

/* Fused q/k/v (matvec.rs:323-345) and gate/up (matvec.rs:407-439) regions:
 * one parallel region over the concatenated rows. */
typedef struct { int kernels, kind; float *out[3]; const uint8_t *w[3]; size_t rows[3]; const void *x; size_t rb, cols; } mv3_ctx;

static void mv3_range(void *c, size_t s, size_t e) {
    mv3_ctx *m = c;
    for (size_t r = s; r < e; r++) {
        int t = 0;
        size_t lr = r;
        while (lr >= m->rows[t]) { lr -= m->rows[t]; t++; }
        m->out[t][lr] = dot_dispatch(m->kernels, m->kind, m->w[t] + lr * m->rb, m->x, m->cols);
    }
}

static void or_matvec_multi(or_pool *p, int kernels, int kind, int n, float *const outs[], const uint8_t *const ws[], const size_t rows[], const void *x, size_t cols) {
    mv3_ctx c;
    memset(&c, 0, sizeof c);
    c.kernels = kernels;
    c.kind = kind;
    c.x = x;
    c.cols = cols;
    c.rb = or_row_bytes(kind, cols);
    size_t total = 0;
    for (int i = 0; i < n; i++) { c.out[i] = outs[i]; c.w[i] = ws[i]; c.rows[i] = rows[i]; total += rows[i]; }
    size_t nth = (size_t)or_pool_threads(p);
    size_t chunk = total / (nth * 8);
    if (chunk < 8) chunk = 8;
    pool_run_chunks(p, total, chunk, mv3_range, &c);
}

typedef struct { int kernels, kind; float *out; const uint8_t *w; const uint8_t *xs; size_t xstride, m, rows, rb, cols; } mm_ctx;

static void mm_range(void *c, size_t s, size_t e) {
    /* matvec.rs:479-522: row blocks of 8, activations 4 at a time through
     * the 1x4 micro-kernel when one exists. */
    mm_ctx *m = c;
    int has4 = m->kernels && (m->kind == AOTK_Q4_0 || m->kind == AOTK_Q5_0 || m->kind == AOTK_Q8_0 || m->kind == AOTK_Q4_K || m->kind == AOTK_Q6_K);
    size_t r0 = s;
    while (r0 < e) {
        size_t r1 = r0 + 8 < e ? r0 + 8 : e;
        size_t i = 0;
        if (has4) {
            for (; i + 4 <= m->m; i += 4) {
                const void *x4[4] = {m->xs + i * m->xstride, m->xs + (i + 1) * m->xstride, m->xs + (i + 2) * m->xstride, m->xs + (i + 3) * m->xstride};
                for (size_t r = r0; r < r1; r++) {
                    float v[4];
                    or_dot_avx2_x4(m->kind, m->w + r * m->rb, x4, m->cols, v);
                    for (int k = 0; k < 4; k++) m->out[(i + k) * m->rows + r] = v[k];
                }
            }
        }
        for (; i < m->m; i++) {
            const void *x = m->xs + i * m->xstride;
            for (size_t r = r0; r < r1; r++) m->out[i * m->rows + r] = dot_dispatch(m->kernels, m->kind, m->w + r * m->rb, x, m->cols);
        }
        r0 = r1;
    }
}

static size_t act_stride(int kind, size_t cols) {
    switch (activation(kind)) {
    case 1: return cols / 32 * sizeof(aotk_block_q8_0);
    case 2: return cols / QK_K * sizeof(aotk_block_q8_k);
    default: return cols * sizeof(float);
    }
}

void or_matmul(or_pool *p, int kernels, int kind, float *out, const uint8_t *w, const void *xs, size_t m, size_t rows, size_t cols) {
    mm_ctx c = {kernels, kind, out, w, xs, act_stride(kind, cols), m, rows, or_row_bytes(kind, cols), cols};
    size_t nth = (size_t)or_pool_threads(p);
    size_t chunk = rows / (nth * 4);
    if (chunk < 8) chunk = 8;
    chunk = (chunk + 7) / 8 * 8;
    pool_run_chunks(p, rows, chunk, mm_range, &c);
}

/* ------------------------------------------------------------------------ */
/* Transformer ops: ops.rs                                                  */
/* ------------------------------------------------------------------------ */

void or_rmsnorm(float *out, const float *x, const float *w, size_t n, float eps) {
    /* ops.rs:7-18 */
    float ss = 0.0f;
    for (size_t i = 0; i < n; i++) ss += x[i] * x[i];
    float r = 1.0f / sqrtf(ss / (float)n + eps);
    for (size_t i = 0; i < n; i++) out[i] = x[i] * r * w[i];
}

void or_rope_cos_sin(float *cs, const float *inv_freq, size_t half, float pos) {
    /* ops.rs:28-34 */
    for (size_t i = 0; i < half; i++) {
        float a = pos * inv_freq[i];
        cs[2 * i] = cosf(a);
        cs[2 * i + 1] = sinf(a);
    }
}

void or_rope(float *x, size_t n_heads, size_t head_dim, size_t rot_dim, const float *cs, int neox) {
    /* ops.rs:40-70 */
    size_t half = rot_dim / 2;
    for (size_t h = 0; h < n_heads; h++) {
        float *v = x + h * head_dim;
        for (size_t i = 0; i < half; i++) {
            float c = cs[2 * i], s = cs[2 * i + 1];
            size_t a = neox ? i : 2 * i, b = neox ? i + half : 2 * i + 1;
            float x0 = v[a], x1 = v[b];
            v[a] = x0 * c - x1 * s;
            v[b] = x0 * s + x1 * c;
        }
    }
}

void or_rmsnorm_heads(float *x, const float *w, size_t n_heads, size_t head_dim, float eps) {
    /* ops.rs:74-87 */
    for (size_t h = 0; h < n_heads; h++) {
        float *v = x + h * head_dim;
        float ss = 0.0f;
        for (size_t i = 0; i < head_dim; i++) ss += v[i] * v[i];
        float r = 1.0f / sqrtf(ss / (float)head_dim + eps);
        for (size_t i = 0; i < head_dim; i++) v[i] = v[i] * r * w[i];
    }
}

void or_softmax(float *x, size_t n) {
    /* ops.rs:98-112 */
    float max = -INFINITY;
    for (size_t i = 0; i < n; i++) max = fmaxf(max, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) { x[i] = expf(x[i] - max); sum += x[i]; }
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; i++) x[i] *= inv;
}

void or_silu_mul(float *h, const float *up, size_t n) {
    /* ops.rs:115-120 */
    for (size_t i = 0; i < n; i++) {
        float v = h[i];
        h[i] = v / (1.0f + expf(-v)) * up[i];
    }
}

float or_gelu(float v) {
    /* ops.rs:124-127 */
    const float k = (float)1.1283791670955126 / (float)1.4142135623730951;
    return 0.5f * v * (1.0f + tanhf(k * (v + 0.044715f * v * v * v)));
}

void or_gelu_mul(float *h, const float *up, size_t n) {
    for (size_t i = 0; i < n; i++) h[i] = or_gelu(h[i]) * up[i];
}

size_t or_window_start(size_t pos, size_t window) {
    /* ops.rs:171-177 */
    return (window > 0 && pos + 1 > window) ? pos + 1 - window : 0;
}

typedef struct {
    float *out; const float *q, *kc, *vc;
    size_t n_head, hd, kv, gqa, ctx, base, pos0, m, window;
    float scale;
} attn_ctx;

static void attn_worker(void *c, int tid, int nth) {
    /* ops.rs:185-218 (`attention`) and :517-556 (`attention_rows`): one task
     * per (row, head); scores, softmax, V mix, all sequential per task. */
    attn_ctx *a = c;
    size_t s, e;
    split_range(a->m * a->n_head, tid, nth, &s, &e);
    float *sc = malloc(sizeof(float) * (a->pos0 + a->m + 1));
    size_t qd = a->n_head * a->hd;
    for (size_t task = s; task < e; task++) {
        size_t i = task / a->n_head, h = task % a->n_head;
        size_t kvh = h / a->gqa;
        size_t n = a->pos0 + i + 1;
        size_t t0 = or_window_start(a->pos0 + i, a->window);
        const float *qh = a->q + i * qd + h * a->hd;
        for (size_t t = t0; t < n; t++) {
            const float *kt = a->kc + a->base + t * a->kv + kvh * a->hd;
            float d = 0.0f;
            for (size_t j = 0; j < a->hd; j++) d += qh[j] * kt[j];
            sc[t - t0] = d * a->scale;
        }
        or_softmax(sc, n - t0);
        float *oh = a->out + i * qd + h * a->hd;
        for (size_t j = 0; j < a->hd; j++) oh[j] = 0.0f;
        for (size_t t = t0; t < n; t++) {
            float w = sc[t - t0];
            const float *vt = a->vc + a->base + t * a->kv + kvh * a->hd;
            for (size_t j = 0; j < a->hd; j++) oh[j] += w * vt[j];
        }
    }
    free(sc);
}

void or_attention(or_pool *p, float *out, const float *q, const float *k_cache, const float *v_cache,
                  size_t n_head, size_t n_kv_head, size_t head_dim, size_t ctx, size_t layer,
                  size_t pos0, size_t m, size_t window) {
    attn_ctx a;
    a.out = out; a.q = q; a.kc = k_cache; a.vc = v_cache;
    a.n_head = n_head; a.hd = head_dim; a.kv = n_kv_head * head_dim; a.gqa = n_head / n_kv_head;
    a.ctx = ctx; a.base = layer * ctx * a.kv; a.pos0 = pos0; a.m = m; a.window = window;
    a.scale = 1.0f / sqrtf((float)head_dim);
    pool_run(p, attn_worker, &a);
}

void or_inv_freq(float *out, size_t rot_dim, float base, const float *factors) {
    /* state.rs:308-319 */
    for (size_t i = 0; i < rot_dim / 2; i++) {
        float f = powf(base, -(2.0f * (float)i) / (float)rot_dim);
        if (factors) f /= factors[i];
        out[i] = f;
    }
}

uint32_t or_argmax(const float *x, size_t n) {
    /* sampler.rs:99-109 */
    size_t best = 0;
    float bv = -INFINITY;
    for (size_t i = 0; i < n; i++) if (x[i] > bv) { bv = x[i]; best = i; }
    return (uint32_t)best;
}

/* ------------------------------------------------------------------------ */
/* Sampler (sampler.rs)                                                     */
/* ------------------------------------------------------------------------ */

uint64_t or_sampler_seed(uint64_t seed) {
    /* splitmix (sampler.rs:113-118), forced odd */
    uint64_t z = seed + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return (z ^ (z >> 31)) | 1ull;
}

static float or_next_f32(uint64_t *rng) {
    /* xorshift64* (sampler.rs:38-45) */
    uint64_t r = *rng;
    r ^= r >> 12;
    r ^= r << 25;
    r ^= r >> 27;
    *rng = r;
    uint64_t v = r * 0x2545F4914F6CDD1Dull;
    return (float)(v >> 40) / (float)(1ull << 24);
}

typedef struct {
    float v;
    uint32_t i;
} or_cand;

/* f32::total_cmp order as an unsigned key (-NaN < -inf < ... < -0 < +0 < ... < +NaN) */
static uint32_t or_total_key(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

static int or_cand_desc(const void *pa, const void *pb) {
    const or_cand *a = (const or_cand *)pa, *b = (const or_cand *)pb;
    uint32_t ka = or_total_key(a->v), kb = or_total_key(b->v);
    if (ka != kb) return ka > kb ? -1 : 1;
    return a->i < b->i ? -1 : (a->i > b->i ? 1 : 0);
}

uint32_t or_sample(const aotk_sampler_config *cfg, uint64_t *rng, float *logits, size_t n, const uint32_t *recent,
                   size_t n_recent) {
    /* repetition penalty (sampler.rs:53-60) */
    if (cfg->repeat_penalty != 1.0f && cfg->repeat_last_n > 0) {
        size_t start = n_recent > cfg->repeat_last_n ? n_recent - cfg->repeat_last_n : 0;
        for (size_t j = start; j < n_recent; j++) {
            float *l = &logits[recent[j]];
            *l = *l > 0.0f ? *l / cfg->repeat_penalty : *l * cfg->repeat_penalty;
        }
    }
    if (cfg->temperature <= 0.0f) return or_argmax(logits, n); /* :61-63 */
    const float inv_t = 1.0f / cfg->temperature;
    or_cand *c = (or_cand *)malloc(n * sizeof(or_cand));
    for (size_t i = 0; i < n; i++) {
        c[i].v = logits[i] * inv_t;
        c[i].i = (uint32_t)i;
    }
    size_t k = cfg->top_k > 0 ? (cfg->top_k < n ? cfg->top_k : n) : n; /* :67 */
    /* select the k largest, then sort them descending (:68-74): one sort
       gives the same k in the same order */
    qsort(c, n, sizeof(or_cand), or_cand_desc);
    const float max = c[0].v;
    float sum = 0.0f;
    for (size_t i = 0; i < k; i++) { /* :75-80 */
        c[i].v = expf(c[i].v - max);
        sum += c[i].v;
    }
    size_t nn = k;
    if (cfg->top_p < 1.0f) { /* :81-91 */
        float acc = 0.0f;
        for (size_t i = 0; i < k; i++) {
            acc += c[i].v / sum;
            if (acc >= cfg->top_p) {
                nn = i + 1;
                break;
            }
        }
        sum = 0.0f;
        for (size_t i = 0; i < nn; i++) sum += c[i].v;
    }
    const float r = or_next_f32(rng) * sum; /* :92-100 */
    float acc = 0.0f;
    uint32_t tok = c[nn - 1].i;
    for (size_t i = 0; i < nn; i++) {
        acc += c[i].v;
        if (acc >= r) {
            tok = c[i].i;
            break;
        }
    }
    free(c);
    return tok;
}

/* ------------------------------------------------------------------------ */
/* Synthetic weights                                                        */
/* ------------------------------------------------------------------------ */

#define SYNTH_SCALE 0x1.1bc77ap-21f /* 0.02 / std of a sum of four U{0..65535} */

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

float or_synth_value(uint64_t seed, uint32_t tensor_index, uint64_t elem) {
    uint64_t key = (seed * 0x9E3779B97F4A7C15ULL) ^ ((uint64_t)(tensor_index + 1) << 40) ^ elem;
    uint64_t z = mix64(key);
    int32_t s = (int32_t)(z & 0xFFFF) + (int32_t)((z >> 16) & 0xFFFF) + (int32_t)((z >> 32) & 0xFFFF) + (int32_t)(z >> 48) - 131070;
    return (float)s * SYNTH_SCALE;
}

void or_e2e_uniform(uint64_t *state, float a, float *out, size_t n) {
    uint64_t s = *state;
    for (size_t i = 0; i < n; i++) {
        s ^= s << 13; /* e2e.rs:84-89 */
        s ^= s >> 7;
        s ^= s << 17;
        float u = (float)(s % 1000001ULL) / 500000.0f - 1.0f; /* :91 */
        out[i] = u * a;
    }
    *state = s;
}

typedef struct { const aotk_tensor *t; uint32_t idx; int is_norm; } synth_item;

static int spec_items(const aotk_model_spec *spec, synth_item *items) {
    int n = 0;
    items[n++] = (synth_item){&spec->token_embd, 0, 0};
    items[n++] = (synth_item){&spec->output_norm, 1, 1};
    if (spec->output.kind != AOTK_KIND_NONE) items[n++] = (synth_item){&spec->output, 2, 0};
    for (uint64_t l = 0; l < spec->dims.n_layer; l++) {
        const aotk_layer *L = &spec->layers[l];
        const aotk_tensor *slots[16] = {&L->attn_norm, &L->wq, &L->wk, &L->wv, &L->wo, &L->ffn_norm, &L->gate, &L->up, &L->down,
                                        &L->bq, &L->bk, &L->bv, &L->q_norm, &L->k_norm, &L->attn_post_norm, &L->ffn_post_norm};
        static const int norm[16] = {1, 0, 0, 0, 0, 1, 0, 0, 0, 0, 0, 0, 1, 1, 1, 1};
        for (int s = 0; s < 16; s++)
            if (slots[s]->kind != AOTK_KIND_NONE) items[n++] = (synth_item){slots[s], (uint32_t)(3 + 16 * l + s), norm[s]};
    }
    return n;
}

typedef struct { synth_item *items; int n; uint64_t seed; uint8_t *blob; } synth_ctx;

static void synth_range(void *c, size_t s, size_t e) {
    /* work unit: (item, row) flattened; rows enumerated item by item */
    synth_ctx *sc = c;
    (void)e;
    for (size_t u = s; u < e; u++) {
        size_t acc = 0;
        int it = 0;
        for (; it < sc->n; it++) {
            if (u < acc + sc->items[it].t->rows) break;
            acc += sc->items[it].t->rows;
        }
        const synth_item *item = &sc->items[it];
        size_t r = u - acc;
        size_t cols = item->t->cols;
        float *tmp = malloc(sizeof(float) * cols);
        for (size_t cc = 0; cc < cols; cc++) {
            float v = or_synth_value(sc->seed, item->idx, (uint64_t)r * cols + cc);
            tmp[cc] = item->is_norm ? 1.0f + v : v;
        }
        or_quantize_row(item->t->kind, tmp, cols, sc->blob + item->t->off + r * or_row_bytes(item->t->kind, cols));
        free(tmp);
    }
}

int or_synth_blob(const aotk_model_spec *spec, uint64_t seed, uint8_t *blob, size_t blob_len, int n_threads) {
    synth_item *items = malloc(sizeof(synth_item) * (3 + 16 * spec->dims.n_layer));
    int n = spec_items(spec, items);
    size_t total = 0;
    for (int i = 0; i < n; i++) {
        if (items[i].t->off + items[i].t->len > blob_len) { free(items); return -1; }
        total += items[i].t->rows;
    }
    memset(blob, 0, blob_len);
    synth_ctx c = {items, n, seed, blob};
    or_pool *p = or_pool_new(n_threads);
    pool_run_chunks(p, total, 64, synth_range, &c);
    or_pool_free(p);
    free(items);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Model: state.rs:251-355 and the emitted forward (emit.rs:167-516)        */
/* ------------------------------------------------------------------------ */

struct or_model {
    aotk_model_spec spec;
    aotk_layer *layers;
    const uint8_t *blob;
    or_pool *pool;
    int kernels;
    size_t ctx, max_batch;
    float *x, *xb, *xb2, *q, *k, *v, *hb, *hb2, *logits, *k_cache, *v_cache;
    aotk_block_q8_0 *aq0;
    aotk_block_q8_k *aqk;
    float *inv_freq, *inv_freq_local, *rope_cs, *rope_cs_local;
    float *bx, *bxb, *bxb2, *bq, *bk, *bv, *bhb, *bhb2, *brope_cs, *brope_cs_local;
    aotk_block_q8_0 *baq0;
    aotk_block_q8_k *baqk;
};

static const float *f32s(const or_model *m, const aotk_tensor *t) { return (const float *)(m->blob + t->off); }
static const uint8_t *tbytes(const or_model *m, const aotk_tensor *t) { return m->blob + t->off; }

static size_t maxz(size_t a, size_t b) { return a > b ? a : b; }

or_model *or_model_new(const aotk_model_spec *spec, const uint8_t *blob, size_t blob_len, size_t ctx, size_t max_batch, int n_threads, int kernels) {
    (void)blob_len;
    or_model *m = calloc(1, sizeof *m);
    m->spec = *spec;
    m->layers = malloc(sizeof(aotk_layer) * spec->dims.n_layer);
    memcpy(m->layers, spec->layers, sizeof(aotk_layer) * spec->dims.n_layer);
    m->spec.layers = m->layers;
    m->blob = blob;
    m->pool = or_pool_new(n_threads);
    m->kernels = kernels;
    m->ctx = ctx;
    if (max_batch < 1) max_batch = 1;
    m->max_batch = max_batch;
    const aotk_dims *d = &spec->dims;
    size_t qd = d->n_head * d->head_dim, kv = d->n_kv_head * d->head_dim;
    size_t big = maxz(maxz(d->dim, qd), d->hidden);
    m->x = calloc(d->dim, 4);
    m->xb = calloc(maxz(d->dim, qd), 4);
    m->xb2 = calloc(d->dim, 4);
    m->q = calloc(qd, 4);
    m->k = calloc(kv, 4);
    m->v = calloc(kv, 4);
    m->hb = calloc(d->hidden, 4);
    m->hb2 = calloc(d->hidden, 4);
    m->logits = calloc(d->vocab, 4);
    m->k_cache = calloc(d->n_layer * ctx * kv, 4);
    m->v_cache = calloc(d->n_layer * ctx * kv, 4);
    m->aq0 = calloc(big / 32 + 1, sizeof(aotk_block_q8_0));
    m->aqk = calloc(big / QK_K + 1, sizeof(aotk_block_q8_k));
    m->inv_freq = calloc(d->rot_dim / 2 + 1, 4);
    const float *ff = spec->rope_freqs.kind != AOTK_KIND_NONE ? (const float *)(blob + spec->rope_freqs.off) : NULL;
    or_inv_freq(m->inv_freq, d->rot_dim, d->rope_base, ff);
    m->rope_cs = calloc(d->rot_dim + 1, 4);
    m->inv_freq_local = calloc(d->rot_dim / 2 + 1, 4);
    m->rope_cs_local = calloc(d->rot_dim + 1, 4);
    if (d->swa_window > 0) or_inv_freq(m->inv_freq_local, d->rot_dim, d->rope_base_local, ff);
    size_t b = max_batch;
    m->bx = calloc(b * d->dim, 4);
    m->bxb = calloc(b * maxz(d->dim, qd), 4);
    m->bxb2 = calloc(b * d->dim, 4);
    m->bq = calloc(b * qd, 4);
    m->bk = calloc(b * kv, 4);
    m->bv = calloc(b * kv, 4);
    m->bhb = calloc(b * d->hidden, 4);
    m->bhb2 = calloc(b * d->hidden, 4);
    m->brope_cs = calloc(b * d->rot_dim + 1, 4);
    m->brope_cs_local = calloc(b * d->rot_dim + 1, 4);
    m->baq0 = calloc(b * (big / 32) + 1, sizeof(aotk_block_q8_0));
    m->baqk = calloc(b * (big / QK_K) + 1, sizeof(aotk_block_q8_k));
    return m;
}

void or_model_free(or_model *m) {
    if (!m) return;
    or_pool_free(m->pool);
    float *fs[] = {m->x, m->xb, m->xb2, m->q, m->k, m->v, m->hb, m->hb2, m->logits, m->k_cache, m->v_cache, m->inv_freq, m->inv_freq_local,
                   m->rope_cs, m->rope_cs_local, m->bx, m->bxb, m->bxb2, m->bq, m->bk, m->bv, m->bhb, m->bhb2, m->brope_cs, m->brope_cs_local};
    for (size_t i = 0; i < sizeof fs / sizeof fs[0]; i++) free(fs[i]);
    free(m->aq0); free(m->aqk); free(m->baq0); free(m->baqk); free(m->layers);
    free(m);
}

const float *or_logits(const or_model *m) { return m->logits; }
float *or_k_cache(or_model *m) { return m->k_cache; }
float *or_v_cache(or_model *m) { return m->v_cache; }

/* emit.rs:131-140 `emit_quantize`: quantize src[..n] into the activation
 * buffers the consumer kinds need. */
static void quantize_for(or_model *m, const float *src, size_t n, const int *kinds, int nk) {
    int need0 = 0, needk = 0;
    for (int i = 0; i < nk; i++) { int a = activation(kinds[i]); need0 |= a == 1; needk |= a == 2; }
    if (need0) or_quantize_q8_0(src, n, m->aq0);
    if (needk) or_quantize_q8_k(src, n, m->aqk);
}

typedef struct { const float *x; size_t n; int q0; aotk_block_q8_0 *o0; aotk_block_q8_k *ok; } qrows_ctx;
static void qrows_range(void *c, size_t s, size_t e) {
    qrows_ctx *q = c;
    if (q->q0) or_quantize_q8_0(q->x + s * 32, (e - s) * 32, q->o0 + s);
    else or_quantize_q8_k(q->x + s * QK_K, (e - s) * QK_K, q->ok + s);
}

/* emit.rs:146-157 `emit_quantize_rows` (quantize_q8_*_par: ops.rs:466-501) */
static void quantize_rows_for(or_model *m, const float *src, size_t total, const int *kinds, int nk) {
    int need0 = 0, needk = 0;
    for (int i = 0; i < nk; i++) { int a = activation(kinds[i]); need0 |= a == 1; needk |= a == 2; }
    if (need0) { qrows_ctx c = {src, total, 1, m->baq0, NULL}; pool_run_chunks(m->pool, total / 32, 32, qrows_range, &c); }
    if (needk) { qrows_ctx c = {src, total, 0, NULL, m->baqk}; pool_run_chunks(m->pool, total / QK_K, 4, qrows_range, &c); }
}

static const void *act_for(or_model *m, int kind, const float *src) {
    switch (activation(kind)) {
    case 1: return m->aq0;
    case 2: return m->aqk;
    default: return src;
    }
}

static const void *bact_for(or_model *m, int kind, const float *src) {
    switch (activation(kind)) {
    case 1: return m->baq0;
    case 2: return m->baqk;
    default: return src;
    }
}

static void mv(or_model *m, const aotk_tensor *t, float *out, const float *src) {
    or_matvec(m->pool, m->kernels, t->kind, out, tbytes(m, t), act_for(m, t->kind, src), t->rows, t->cols);
}

static void mm(or_model *m, const aotk_tensor *t, float *out, const float *src, size_t n) {
    or_matmul(m->pool, m->kernels, t->kind, out, tbytes(m, t), bact_for(m, t->kind, src), n, t->rows, t->cols);
}

static void add_inplace(float *x, const float *y, size_t n) {
    for (size_t i = 0; i < n; i++) x[i] += y[i];
}

static void layer_decode(or_model *m, size_t li, size_t pos) {
    /* emit.rs:243-333 */
    const aotk_dims *d = &m->spec.dims;
    const aotk_flags *f = &m->spec.flags;
    const aotk_layer *l = &m->layers[li];
    size_t dim = d->dim, qd = d->n_head * d->head_dim, kv = d->n_kv_head * d->head_dim;
    const float *cs = l->local_attn ? m->rope_cs_local : m->rope_cs;
    size_t window = l->local_attn ? d->swa_window : 0;
    or_rmsnorm(m->xb, m->x, f32s(m, &l->attn_norm), dim, d->eps);
    int k3[3] = {l->wq.kind, l->wk.kind, l->wv.kind};
    quantize_for(m, m->xb, dim, k3, 3);
    if (l->wq.kind == l->wk.kind && l->wk.kind == l->wv.kind && activation(l->wq.kind) != 0) {
        float *outs[3] = {m->q, m->k, m->v};
        const uint8_t *ws[3] = {tbytes(m, &l->wq), tbytes(m, &l->wk), tbytes(m, &l->wv)};
        size_t rows[3] = {l->wq.rows, l->wk.rows, l->wv.rows};
        or_matvec_multi(m->pool, m->kernels, l->wq.kind, 3, outs, ws, rows, act_for(m, l->wq.kind, m->xb), l->wq.cols);
    } else {
        mv(m, &l->wq, m->q, m->xb);
        mv(m, &l->wk, m->k, m->xb);
        mv(m, &l->wv, m->v, m->xb);
    }
    if (f->qkv_bias) {
        add_inplace(m->q, f32s(m, &l->bq), qd);
        add_inplace(m->k, f32s(m, &l->bk), kv);
        add_inplace(m->v, f32s(m, &l->bv), kv);
    }
    if (f->qk_norm) {
        or_rmsnorm_heads(m->q, f32s(m, &l->q_norm), d->n_head, d->head_dim, d->eps);
        or_rmsnorm_heads(m->k, f32s(m, &l->k_norm), d->n_kv_head, d->head_dim, d->eps);
    }
    or_rope(m->q, d->n_head, d->head_dim, d->rot_dim, cs, f->rope_neox);
    or_rope(m->k, d->n_kv_head, d->head_dim, d->rot_dim, cs, f->rope_neox);
    size_t at = (li * m->ctx + pos) * kv;
    memcpy(m->k_cache + at, m->k, kv * 4);
    memcpy(m->v_cache + at, m->v, kv * 4);
    or_attention(m->pool, m->xb, m->q, m->k_cache, m->v_cache, d->n_head, d->n_kv_head, d->head_dim, m->ctx, li, pos, 1, window);
    int ko = l->wo.kind;
    quantize_for(m, m->xb, qd, &ko, 1);
    mv(m, &l->wo, m->xb2, m->xb);
    if (f->post_norms) {
        or_rmsnorm(m->xb, m->xb2, f32s(m, &l->attn_post_norm), dim, d->eps);
        add_inplace(m->x, m->xb, dim);
    } else {
        add_inplace(m->x, m->xb2, dim);
    }
    or_rmsnorm(m->xb, m->x, f32s(m, &l->ffn_norm), dim, d->eps);
    int k2[2] = {l->gate.kind, l->up.kind};
    quantize_for(m, m->xb, dim, k2, 2);
    if (l->gate.kind == l->up.kind && activation(l->gate.kind) != 0) {
        float *outs[2] = {m->hb, m->hb2};
        const uint8_t *ws[2] = {tbytes(m, &l->gate), tbytes(m, &l->up)};
        size_t rows[2] = {l->gate.rows, l->up.rows};
        or_matvec_multi(m->pool, m->kernels, l->gate.kind, 2, outs, ws, rows, act_for(m, l->gate.kind, m->xb), l->gate.cols);
    } else {
        mv(m, &l->gate, m->hb, m->xb);
        mv(m, &l->up, m->hb2, m->xb);
    }
    if (f->gelu) or_gelu_mul(m->hb, m->hb2, d->hidden);
    else or_silu_mul(m->hb, m->hb2, d->hidden);
    int kd = l->down.kind;
    quantize_for(m, m->hb, d->hidden, &kd, 1);
    mv(m, &l->down, m->xb2, m->hb);
    if (f->post_norms) {
        or_rmsnorm(m->xb, m->xb2, f32s(m, &l->ffn_post_norm), dim, d->eps);
        add_inplace(m->x, m->xb, dim);
    } else {
        add_inplace(m->x, m->xb2, dim);
    }
}

static const aotk_tensor *out_tensor(const or_model *m) {
    return m->spec.output.kind != AOTK_KIND_NONE ? &m->spec.output : &m->spec.token_embd;
}

static void logits_from(or_model *m, const float *x) {
    const aotk_dims *d = &m->spec.dims;
    or_rmsnorm(m->xb, x, f32s(m, &m->spec.output_norm), d->dim, d->eps);
    int ko = out_tensor(m)->kind;
    quantize_for(m, m->xb, d->dim, &ko, 1);
    mv(m, out_tensor(m), m->logits, m->xb);
}

int or_forward(or_model *m, uint32_t token, size_t pos, int want_logits) {
    /* emit.rs:466-486 */
    const aotk_dims *d = &m->spec.dims;
    if (token >= d->vocab || pos >= m->ctx) return -1;
    const aotk_tensor *e = &m->spec.token_embd;
    or_dequant_row(e->kind, tbytes(m, e) + (size_t)token * or_row_bytes(e->kind, e->cols), m->x, d->dim);
    if (m->spec.flags.embd_scale) {
        float s = sqrtf((float)d->dim);
        for (size_t i = 0; i < d->dim; i++) m->x[i] *= s;
    }
    or_rope_cos_sin(m->rope_cs, m->inv_freq, d->rot_dim / 2, (float)pos / d->rope_scale);
    if (d->swa_window > 0) or_rope_cos_sin(m->rope_cs_local, m->inv_freq_local, d->rot_dim / 2, (float)pos / d->rope_scale_local);
    for (size_t l = 0; l < d->n_layer; l++) layer_decode(m, l, pos);
    if (want_logits) logits_from(m, m->x);
    return 0;
}

typedef struct { float *out; const float *x, *w; size_t n; float eps; } rows_ctx;
static void rmsnorm_rows_range(void *c, size_t s, size_t e) {
    rows_ctx *r = c;
    for (size_t i = s; i < e; i++) or_rmsnorm(r->out + i * r->n, r->x + i * r->n, r->w, r->n, r->eps);
}
static void rmsnorm_rows(or_model *m, float *out, const float *x, const float *w, size_t n, size_t rows, float eps) {
    /* ops.rs:361-366, :419-432 */
    rows_ctx c = {out, x, w, n, eps};
    pool_run_chunks(m->pool, rows, 1, rmsnorm_rows_range, &c);
}

static void layer_batch(or_model *m, size_t li, size_t pos0, size_t n) {
    /* emit.rs:167-237 */
    const aotk_dims *d = &m->spec.dims;
    const aotk_flags *f = &m->spec.flags;
    const aotk_layer *l = &m->layers[li];
    size_t dim = d->dim, hidden = d->hidden, qd = d->n_head * d->head_dim, kv = d->n_kv_head * d->head_dim;
    const float *cs = l->local_attn ? m->brope_cs_local : m->brope_cs;
    size_t window = l->local_attn ? d->swa_window : 0;
    rmsnorm_rows(m, m->bxb, m->bx, f32s(m, &l->attn_norm), dim, n, d->eps);
    int k3[3] = {l->wq.kind, l->wk.kind, l->wv.kind};
    quantize_rows_for(m, m->bxb, n * dim, k3, 3);
    mm(m, &l->wq, m->bq, m->bxb, n);
    mm(m, &l->wk, m->bk, m->bxb, n);
    mm(m, &l->wv, m->bv, m->bxb, n);
    if (f->qkv_bias) {
        for (size_t i = 0; i < n; i++) {
            add_inplace(m->bq + i * qd, f32s(m, &l->bq), qd);
            add_inplace(m->bk + i * kv, f32s(m, &l->bk), kv);
            add_inplace(m->bv + i * kv, f32s(m, &l->bv), kv);
        }
    }
    if (f->qk_norm) {
        or_rmsnorm_heads(m->bq, f32s(m, &l->q_norm), n * d->n_head, d->head_dim, d->eps);
        or_rmsnorm_heads(m->bk, f32s(m, &l->k_norm), n * d->n_kv_head, d->head_dim, d->eps);
    }
    for (size_t i = 0; i < n; i++) {
        or_rope(m->bq + i * qd, d->n_head, d->head_dim, d->rot_dim, cs + i * d->rot_dim, f->rope_neox);
        or_rope(m->bk + i * kv, d->n_kv_head, d->head_dim, d->rot_dim, cs + i * d->rot_dim, f->rope_neox);
    }
    size_t at = (li * m->ctx + pos0) * kv;
    memcpy(m->k_cache + at, m->bk, n * kv * 4);
    memcpy(m->v_cache + at, m->bv, n * kv * 4);
    or_attention(m->pool, m->bxb, m->bq, m->k_cache, m->v_cache, d->n_head, d->n_kv_head, d->head_dim, m->ctx, li, pos0, n, window);
    int ko = l->wo.kind;
    quantize_rows_for(m, m->bxb, n * qd, &ko, 1);
    mm(m, &l->wo, m->bxb2, m->bxb, n);
    if (f->post_norms) {
        rmsnorm_rows(m, m->bxb, m->bxb2, f32s(m, &l->attn_post_norm), dim, n, d->eps);
        add_inplace(m->bx, m->bxb, n * dim);
    } else {
        add_inplace(m->bx, m->bxb2, n * dim);
    }
    rmsnorm_rows(m, m->bxb, m->bx, f32s(m, &l->ffn_norm), dim, n, d->eps);
    int k2[2] = {l->gate.kind, l->up.kind};
    quantize_rows_for(m, m->bxb, n * dim, k2, 2);
    mm(m, &l->gate, m->bhb, m->bxb, n);
    mm(m, &l->up, m->bhb2, m->bxb, n);
    if (f->gelu) or_gelu_mul(m->bhb, m->bhb2, n * hidden);
    else or_silu_mul(m->bhb, m->bhb2, n * hidden);
    int kd = l->down.kind;
    quantize_rows_for(m, m->bhb, n * hidden, &kd, 1);
    mm(m, &l->down, m->bxb2, m->bhb, n);
    if (f->post_norms) {
        rmsnorm_rows(m, m->bxb, m->bxb2, f32s(m, &l->ffn_post_norm), dim, n, d->eps);
        add_inplace(m->bx, m->bxb, n * dim);
    } else {
        add_inplace(m->bx, m->bxb2, n * dim);
    }
}

int or_forward_batch(or_model *m, const uint32_t *tokens, size_t n, size_t pos0, int want_logits) {
    /* emit.rs:491-516 */
    const aotk_dims *d = &m->spec.dims;
    if (n < 1 || n > m->max_batch || pos0 + n > m->ctx) return -1;
    const aotk_tensor *e = &m->spec.token_embd;
    for (size_t i = 0; i < n; i++) {
        if (tokens[i] >= d->vocab) return -1;
        or_dequant_row(e->kind, tbytes(m, e) + (size_t)tokens[i] * or_row_bytes(e->kind, e->cols), m->bx + i * d->dim, d->dim);
    }
    if (m->spec.flags.embd_scale) {
        float s = sqrtf((float)d->dim);
        for (size_t i = 0; i < n * d->dim; i++) m->bx[i] *= s;
    }
    for (size_t i = 0; i < n; i++) {
        or_rope_cos_sin(m->brope_cs + i * d->rot_dim, m->inv_freq, d->rot_dim / 2, (float)(pos0 + i) / d->rope_scale);
        if (d->swa_window > 0)
            or_rope_cos_sin(m->brope_cs_local + i * d->rot_dim, m->inv_freq_local, d->rot_dim / 2, (float)(pos0 + i) / d->rope_scale_local);
    }
    for (size_t l = 0; l < d->n_layer; l++) layer_batch(m, l, pos0, n);
    if (want_logits) logits_from(m, m->bx + (n - 1) * d->dim);
    return 0;
}
