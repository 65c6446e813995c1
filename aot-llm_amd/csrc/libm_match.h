/* libm_match.h - expf / tanhf returning exactly what the host C library
 * returns, on the host and on gfx950.
 *
 * The reference computes softmax, SiLU and GELU with Rust's f32::exp /
 * f32::tanh, which call the platform libm (glibc expf / tanhf on Linux,
 * crates/aot-kernels/src/ops.rs:98-134). One ulp of difference there can flip
 * an int8 activation rounding downstream, so the device restates the
 * published algorithms glibc uses (named at each function below) with the
 * same IEEE operation sequence. gen_libm_tables.c runs this same source on
 * the host against the host libm over all 2^32 inputs and writes the few
 * inputs where they still differ to libm_tables.h; aotk_expf / aotk_tanhf in
 * device.hpp consult that table.
 */
#ifndef AOTK_LIBM_MATCH_H
#define AOTK_LIBM_MATCH_H

#include <stdint.h>

#ifdef __HIPCC__
#define LM_FN __host__ __device__ static inline
#else
#include <math.h>
#include <string.h>
#define LM_FN static inline
#endif

LM_FN double lm_fma(double a, double b, double c) { return fma(a, b, c); }

LM_FN double lm_u2d(uint64_t u) {
    double d;
#ifdef __HIPCC__
    d = __builtin_bit_cast(double, u);
#else
    memcpy(&d, &u, 8);
#endif
    return d;
}

LM_FN uint32_t lm_f2u(float f) {
#ifdef __HIPCC__
    return __builtin_bit_cast(uint32_t, f);
#else
    uint32_t u; memcpy(&u, &f, 4); return u;
#endif
}
LM_FN float lm_u2f(uint32_t u) {
#ifdef __HIPCC__
    return __builtin_bit_cast(float, u);
#else
    float f; memcpy(&f, &u, 4); return f;
#endif
}
LM_FN uint64_t lm_d2u(double d) {
#ifdef __HIPCC__
    return __builtin_bit_cast(uint64_t, d);
#else
    uint64_t u; memcpy(&u, &d, 8); return u;
#endif
}

/* ---- expf: the table-driven method of glibc >= 2.27 (Szabolcs Nagy's
 * exp2f-based expf from ARM optimized-routines): z = x * 32/ln2 rounded to
 * k/32 with a 1.5*2^52 shift, 2^(k/32) from a 32-entry table of
 * 2^(i/32) (nearest doubles, exponent bits pre-subtracted), and a cubic for
 * 2^(r/32) evaluated in double. x86-64 glibc selects its FMA build on FMA
 * hardware, so the polynomial steps are fused. */
#ifdef __HIPCC__
__device__ __constant__ static const uint64_t lm_exp2f_tab_dev[32] = {
0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL};
#endif
static const uint64_t lm_exp2f_tab_host[32] = {
0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL};

/* tab: the 32-entry table (a copy of it, e.g. in LDS on the device) */
LM_FN float lm_expf_tab(float x, const uint64_t *tab) {
    const double invln2n = 0x1.71547652b82fep+0 * 32;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32, c2 = 0x1.62e42ff0c52d6p-1 / 32;
    uint32_t abstop = (lm_f2u(x) >> 20) & 0x7ff;
    if (abstop >= ((lm_f2u(88.0f) >> 20) & 0x7ff)) {
        if (lm_f2u(x) == lm_f2u(-INFINITY)) return 0.0f;
        if (abstop >= ((lm_f2u(INFINITY) >> 20) & 0x7ff)) return x + x;
        if (x > 0x1.62e42ep6f) return INFINITY;
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    double xd = (double)x;
    double z = invln2n * xd;
    double kd = z + shift;
    uint64_t ki = lm_d2u(kd);
    kd -= shift;
    double r = z - kd;
    uint64_t t = tab[ki % 32];
    t += ki << (52 - 5);
    double s = lm_u2d(t);
    double zz = lm_fma(c0, r, c1);
    double r2 = r * r;
    double y = lm_fma(c2, r, 1.0);
    y = lm_fma(zz, r2, y);
    y = y * s;
    return (float)y;
}

LM_FN float lm_expf(float x) {
#ifdef __HIP_DEVICE_COMPILE__
    return lm_expf_tab(x, lm_exp2f_tab_dev);
#else
    return lm_expf_tab(x, lm_exp2f_tab_host);
#endif
}

/* ---- tanhf: fdlibm's s_tanhf.c / s_expm1f.c (Sun Microsystems, the
 * float-precision algorithm glibc ships as tanhf/expm1f), restated. */
LM_FN float lm_expm1f(float x) {
    const float huge = 1.0e+30f, tiny = 1.0e-30f, o_threshold = 8.8721679688e+01f;
    const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f, invln2 = 1.4426950216e+00f;
    const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f, Q4 = 4.0082177293e-06f,
                Q5 = -2.0109921195e-07f;
    float y, hi, lo, c = 0.0f, t, e, hxs, hfx, r1;
    int32_t k;
    uint32_t hx = lm_f2u(x);
    uint32_t xsb = hx & 0x80000000u;
    y = xsb == 0 ? x : -x;
    hx &= 0x7fffffffu;
    if (hx >= 0x4195b844u) {
        if (hx >= 0x42b17218u) {
            if (hx > 0x7f800000u) return x + x;
            if (hx == 0x7f800000u) return xsb == 0 ? x : -1.0f;
            if (x > o_threshold) return huge * huge;
        }
        if (xsb != 0) return tiny - 1.0f;
    }
    if (hx > 0x3eb17218u) {
        if (hx < 0x3F851592u) {
            if (xsb == 0) { hi = x - ln2_hi; lo = ln2_lo; k = 1; }
            else { hi = x + ln2_hi; lo = -ln2_lo; k = -1; }
        } else {
            k = (int32_t)(invln2 * x + (xsb == 0 ? 0.5f : -0.5f));
            t = (float)k;
            hi = x - t * ln2_hi;
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000u) {
        t = huge + x;
        return x - (t - (huge + x));
    } else {
        k = 0;
    }
    hfx = 0.5f * x;
    hxs = x * hfx;
    r1 = 1.0f + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
    t = 3.0f - r1 * hfx;
    e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = (x * (e - c) - c);
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) {
        if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
        return 1.0f + 2.0f * (x - e);
    }
    if (k <= -2 || k > 56) {
        y = 1.0f - (e - x);
        y = lm_u2f(lm_f2u(y) + ((uint32_t)k << 23));
        return y - 1.0f;
    }
    if (k < 23) {
        t = lm_u2f(0x3f800000u - (0x1000000u >> k));
        y = t - (e - x);
        y = lm_u2f(lm_f2u(y) + ((uint32_t)k << 23));
    } else {
        t = lm_u2f((uint32_t)(0x7f - k) << 23);
        y = x - (e + t);
        y += 1.0f;
        y = lm_u2f(lm_f2u(y) + ((uint32_t)k << 23));
    }
    return y;
}

LM_FN float lm_tanhf(float x) {
    float t, z;
    int32_t jx = (int32_t)lm_f2u(x);
    int32_t ix = jx & 0x7fffffff;
    if (ix >= 0x7f800000) return jx >= 0 ? 1.0f / x + 1.0f : 1.0f / x - 1.0f;
    if (ix < 0x41b00000) {
        if (ix == 0) return x;
        if (ix < 0x24000000) return x * (1.0f + x);
        if (ix >= 0x3f800000) {
            t = lm_expm1f(2.0f * fabsf(x));
            z = 1.0f - 2.0f / (t + 2.0f);
        } else {
            t = lm_expm1f(-2.0f * fabsf(x));
            z = -t / (t + 2.0f);
        }
    } else {
        z = 1.0f - 1.0e-30f;
    }
    return jx >= 0 ? z : -z;
}

#endif
