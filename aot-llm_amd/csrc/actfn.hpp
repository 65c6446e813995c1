// actfn.hpp - device helpers shared by the matvec and the ops kernels: the
// activation quantizers of one 256-value block held by a wave, and the GLU
// activations.
#pragma once

#include "device.hpp"
#include "internal.hpp"

namespace aotk {

// DPP lane exchanges within rows of 16 lanes (all sources valid):
// quad_perm xor 1 / xor 2, row_half_mirror (lane i <-> 7 - i of each 8),
// row_mirror (lane i <-> 15 - i). After xor 1 and xor 2 a quad holds one
// value, so the mirrors then pair whole quads / half-rows like xor 4 / xor 8.
template <int CTRL>
__device__ __forceinline__ int dppx_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false); }
template <int CTRL>
__device__ __forceinline__ float dppx_f(float v) { return __int_as_float(dppx_i<CTRL>(__float_as_int(v))); }
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;

// One lane's share of a Q8_K block (quant.rs:248-283) of 256 values held 4
// per lane (element 4*lane + k) of a wave: the 4 packed quants, the sum of
// the lane's quad of 4 lanes (lanes 4j hold bsums[j]) and the block scale d.
struct Q8KLane {
    uint32_t packed;
    int quad_sum;
    float d;
};
// |f| as an integer of the same order; NaN maps to 0, below every value,
// as the reference's strict '>' scan from 0 never picks a NaN.
__device__ __forceinline__ uint32_t mag_bits(float f) {
    const uint32_t b = __float_as_uint(f) & 0x7FFFFFFFu;
    return b > 0x7F800000u ? 0u : b;
}
template <int CTRL>
__device__ __forceinline__ uint32_t dppx_u(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}

__device__ __forceinline__ Q8KLane q8k_lane(const float v[4], int lane) {
    // the largest magnitude over the wave, as ordered integers
    uint32_t m[4];
#pragma unroll
    for (int k = 0; k < 4; k++) m[k] = mag_bits(v[k]);
    uint32_t a = max(max(m[0], m[1]), max(m[2], m[3]));
    a = max(a, dppx_u<DPP_XOR1>(a));
    a = max(a, dppx_u<DPP_XOR2>(a));
    a = max(a, dppx_u<DPP_HALF_MIRROR>(a));
    a = max(a, dppx_u<DPP_MIRROR>(a));
    const uint32_t amax = max(max((uint32_t)__builtin_amdgcn_readlane((int)a, 0), (uint32_t)__builtin_amdgcn_readlane((int)a, 16)),
                              max((uint32_t)__builtin_amdgcn_readlane((int)a, 32), (uint32_t)__builtin_amdgcn_readlane((int)a, 48)));
    // its first index 4 * lane + k: the lowest lane holding it, then that
    // lane's lowest k
    const int kl = m[0] == amax ? 0 : (m[1] == amax ? 1 : (m[2] == amax ? 2 : (m[3] == amax ? 3 : 4)));
    const unsigned long long hit = __ballot(kl < 4);
    const int src_lane = hit ? (int)__builtin_ctzll(hit) : 0;
    const int sk = __builtin_amdgcn_readlane(kl, src_lane);
    const float pick = sk == 0 ? v[0] : (sk == 1 ? v[1] : (sk == 2 ? v[2] : v[3]));
    const float max = readlane_f(pick, src_lane);
    Q8KLane r;
    r.packed = 0;
    int sum = 0;
    r.d = 0.0f;
    if (amax != 0u) {  // all zeros (or all NaN: the scan never moves off 0) give a zero block
        const float iscale = -127.0f / max;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            // Rust's saturating `as i32` (NaN -> 0) is the conversion's own behaviour
            int t = (int)roundf(iscale * v[k]);
            t = t > 127 ? 127 : t;
            r.packed |= (uint32_t)(t & 0xFF) << (8 * k);
            sum += (int8_t)t;
        }
        r.d = 1.0f / iscale;
    }
    sum += dppx_i<DPP_XOR1>(sum);
    sum += dppx_i<DPP_XOR2>(sum);
    r.quad_sum = sum;
    return r;
}

// One lane's share of the 8 Q8_0 blocks (quant.rs:231-245) of 256 values
// held 4 per lane (element 4*lane + k; lanes 8j..8j+7 hold block j): the
// packed quants, the quants themselves and the block scale d.
__device__ __forceinline__ uint32_t q80_lane(const float v[4], int (&qv)[4], float &d) {
    float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    amax = fmaxf(amax, dppx_f<DPP_XOR1>(amax));
    amax = fmaxf(amax, dppx_f<DPP_XOR2>(amax));
    amax = fmaxf(amax, dppx_f<DPP_HALF_MIRROR>(amax));
    d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint32_t packed = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        qv[k] = clampi(round_i(v[k] * id), -127, 127);
        packed |= (uint32_t)(qv[k] & 0xFF) << (8 * k);
    }
    return packed;
}

// Quantize 256 values held 4 per lane (element 4*lane + k) of one wave into
// the Q8_K block `blk` (quant.rs:248-283) and/or the 8 Q8_0 blocks
// 8*blk .. 8*blk+7 (quant.rs:231-245).
__device__ __forceinline__ void quant256(const float v[4], int lane, size_t blk, ActQ8K q8k, ActQ8_0 q80) {
    if (q8k.qs) {
        const Q8KLane r = q8k_lane(v, lane);
        ((uint32_t *)(q8k.qs + blk * 256))[lane] = r.packed;
        if (q8k.qt) {  // the tiled copy: elements 4*lane .. +3 are one aligned 4-byte run there
            const size_t v = (size_t)q8k.tok + blk / q8k.nbt;
            *(uint32_t *)(q8k.qt + q8k_tiled_off(v, (int)(blk % q8k.nbt), q8k.nbt, 4 * lane)) = r.packed;
        }
        if ((lane & 3) == 0) q8k.bsums[blk * 16 + lane / 4] = (int16_t)r.quad_sum;
        if (lane == 0) q8k.d[blk] = r.d;
    }
    if (q80.qs) {
        int qv[4];
        float d;
        const uint32_t packed = q80_lane(v, qv, d);
        ((uint32_t *)(q80.qs + blk * 256))[lane] = packed;
        if (q80.xh) {  // batches: the quants as f16 for the matrix-core products
            const uint32_t h01 = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)qv[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)qv[1]) << 16);
            const uint32_t h23 = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)qv[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)qv[3]) << 16);
            ((uint2 *)(q80.xh + blk * 256))[lane] = make_uint2(h01, h23);
        }
        if ((lane & 7) == 0) q80.d[blk * 8 + lane / 8] = d;
    }
}

__device__ __forceinline__ float silu_f(float v, float b) { return v / (1.0f + aotk_expf(-v)) * b; }
__device__ __forceinline__ float gelu_f(float v) {
    const float k = (float)1.1283791670955126 / (float)1.4142135623730951;
    return 0.5f * v * (1.0f + aotk_tanhf(k * (v + 0.044715f * v * v * v)));
}


}  // namespace aotk
