// formats.hpp - element access of the device weight layouts (plane layout of
// DevWeight), shared by the dequantizer and the embedding lookup.
#pragma once

#include "device.hpp"
#include "internal.hpp"

namespace aotk {

struct WView {
    const uint8_t *p0, *p1, *p2;
    size_t nb, rb;
};

// Value of element c of row r: quant.rs:300-443 with the same two roundings.
template <int KIND>
__device__ __forceinline__ float dequant_elem(const WView &w, size_t r, size_t c) {
    if (KIND == AOTK_F32) return ((const float *)(w.p0 + r * w.rb))[c];
    if (KIND == AOTK_F16) return f16_to_f32(((const uint16_t *)(w.p0 + r * w.rb))[c]);
    if (KIND == AOTK_BF16) return bf16_to_f32(((const uint16_t *)(w.p0 + r * w.rb))[c]);
    if (KIND == AOTK_Q4_0 || KIND == AOTK_Q5_0 || KIND == AOTK_Q8_0) {
        size_t blk = r * w.nb + c / 32;
        int j = (int)(c % 32);
        float d = f16_to_f32(((const uint16_t *)w.p1)[blk]);
        if (KIND == AOTK_Q8_0) return (float)(int8_t)w.p0[blk * 32 + j] * d;
        uint8_t q = w.p0[blk * 16 + (j & 15)];
        int v = j < 16 ? (q & 0xF) : (q >> 4);
        if (KIND == AOTK_Q4_0) return (float)(v - 8) * d;
        uint32_t qh = ((const uint32_t *)w.p2)[blk];
        v |= (int)((qh >> j) & 1u) << 4;
        return (float)(v - 16) * d;
    }
    if (KIND == AOTK_Q4_K || KIND == AOTK_Q5_K) {
        const uint8_t *rowp = w.p0 + r * w.rb;
        const size_t sb = c / 256, nb = w.nb;
        auto B = [&](int off) { return rowp[kq_off(off, sb, nb)]; };
        int e = (int)(c % 256);
        int j = e / 64, hi = (e % 64) / 32, l = e % 32;
        const uint32_t *h = (const uint32_t *)(rowp + kq_off(0, sb, nb));  // bytes [0,16) are one chunk
        float d = f16_to_f32(h[0] & 0xFFFF), dmin = f16_to_f32(h[0] >> 16);
        int sc, m;
        scale_min_k4(2 * j + hi, h[1], h[2], h[3], sc, m);
        float d1 = d * (float)sc, m1 = dmin * (float)m;
        int q;
        if (KIND == AOTK_Q4_K) {
            uint8_t qb = B(16 + 32 * j + l);
            q = hi ? (qb >> 4) : (qb & 0xF);
        } else {
            uint8_t qb = B(48 + 32 * j + l);
            q = hi ? (qb >> 4) : (qb & 0xF);
            if (B(16 + l) & (1u << (2 * j + hi))) q += 16;
        }
        return d1 * (float)q - m1;
    }
    // Q6_K
    const size_t sb = c / 256, nb = w.nb, blk = r * nb + sb;
    const uint8_t *rowp = w.p0 + r * nb * 208;
    auto B = [&](int off) { return rowp[kq_off(off, sb, nb)]; };
    float d = f16_to_f32(((const uint16_t *)w.p1)[blk]);
    int e = (int)(c % 256);
    int n = e / 128, t = e % 128, quarter = t / 32, l = t % 32;
    int lo = (quarter & 1) ? B(64 * n + l + 32) : B(64 * n + l);
    lo = (quarter >= 2) ? (lo >> 4) : (lo & 0xF);
    int q = (lo | (((B(128 + 32 * n + l) >> (2 * quarter)) & 3) << 4)) - 32;
    return d * (float)(int8_t)B(192 + 8 * n + l / 16 + 2 * quarter) * (float)q;
}


#define AOTK_KIND_SWITCH(kind, F)      \
    switch (kind) {                    \
    case AOTK_F32: F(AOTK_F32); break; \
    case AOTK_F16: F(AOTK_F16); break; \
    case AOTK_BF16: F(AOTK_BF16); break; \
    case AOTK_Q4_0: F(AOTK_Q4_0); break; \
    case AOTK_Q5_0: F(AOTK_Q5_0); break; \
    case AOTK_Q8_0: F(AOTK_Q8_0); break; \
    case AOTK_Q4_K: F(AOTK_Q4_K); break; \
    case AOTK_Q5_K: F(AOTK_Q5_K); break; \
    case AOTK_Q6_K: F(AOTK_Q6_K); break; \
    default: break;                    \
    }


inline WView view_of(const DevWeight &w) {
    WView v;
    v.p0 = w.plane[0];
    v.p1 = w.plane[1];
    v.p2 = w.plane[2];
    v.nb = w.nb;
    v.rb = row_bytes(w.kind, w.cols);
    return v;
}

}  // namespace aotk
