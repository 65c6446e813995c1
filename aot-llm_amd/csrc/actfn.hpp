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

// (|value|, index) reduction keeping the largest value, the smallest index
// among equals (the first index of the maximum).
template <int CTRL>
__device__ __forceinline__ void amax_step(float &amax, int &idx) {
    const float oa = dppx_f<CTRL>(amax);
    const int oi = dppx_i<CTRL>(idx);
    if (oa > amax || (oa == amax && oi < idx)) {
        amax = oa;
        idx = oi;
    }
}

// One lane's share of a Q8_K block (quant.rs:248-283) of 256 values held 4
// per lane (element 4*lane + k) of a wave: the 4 packed quants, the sum of
// the lane's quad of 4 lanes (lanes 4j hold bsums[j]) and the block scale d.
struct Q8KLane {
    uint32_t packed;
    int quad_sum;
    float d;
};
__device__ __forceinline__ Q8KLane q8k_lane(const float v[4], int lane) {
    float amax = 0.0f;
    int idx = 0x7fffffff;
    for (int k = 0; k < 4; k++) {
        float a = fabsf(v[k]);
        if (a > amax) { amax = a; idx = lane * 4 + k; }
    }
    amax_step<DPP_XOR1>(amax, idx);
    amax_step<DPP_XOR2>(amax, idx);
    amax_step<DPP_HALF_MIRROR>(amax, idx);
    amax_step<DPP_MIRROR>(amax, idx);
    // the four rows of 16 lanes, in index order
    {
        float ra = readlane_f(amax, 0);
        int ri = __builtin_amdgcn_readlane(idx, 0);
#pragma unroll
        for (int r = 1; r < 4; r++) {
            const float oa = readlane_f(amax, 16 * r);
            const int oi = __builtin_amdgcn_readlane(idx, 16 * r);
            if (oa > ra || (oa == ra && oi < ri)) {
                ra = oa;
                ri = oi;
            }
        }
        amax = ra;
        idx = ri;
    }
    const int src_lane = (idx == 0x7fffffff) ? 0 : idx >> 2, sk = idx & 3;
    const float c0 = readlane_f(v[0], src_lane), c1 = readlane_f(v[1], src_lane);
    const float c2 = readlane_f(v[2], src_lane), c3 = readlane_f(v[3], src_lane);
    float max = sk == 0 ? c0 : (sk == 1 ? c1 : (sk == 2 ? c2 : c3));
    Q8KLane r;
    r.packed = 0;
    int sum = 0;
    r.d = 0.0f;
    if (amax != 0.0f) {
        float iscale = -127.0f / max;
        for (int k = 0; k < 4; k++) {
            int t = round_i(iscale * v[k]);
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

// Quantize 256 values held 4 per lane (element 4*lane + k) of one wave into
// the Q8_K block `blk` (quant.rs:248-283) and/or the 8 Q8_0 blocks
// 8*blk .. 8*blk+7 (quant.rs:231-245).
__device__ __forceinline__ void quant256(const float v[4], int lane, size_t blk, ActQ8K q8k, ActQ8_0 q80) {
    if (q8k.qs) {
        const Q8KLane r = q8k_lane(v, lane);
        ((uint32_t *)(q8k.qs + blk * 256))[lane] = r.packed;
        if ((lane & 3) == 0) q8k.bsums[blk * 16 + lane / 4] = (int16_t)r.quad_sum;
        if (lane == 0) q8k.d[blk] = r.d;
    }
    if (q80.qs) {
        float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        amax = fmaxf(amax, dppx_f<DPP_XOR1>(amax));
        amax = fmaxf(amax, dppx_f<DPP_XOR2>(amax));
        amax = fmaxf(amax, dppx_f<DPP_HALF_MIRROR>(amax));
        float d = amax / 127.0f;
        float id = d != 0.0f ? 1.0f / d : 0.0f;
        uint32_t packed = 0;
        for (int k = 0; k < 4; k++) packed |= (uint32_t)(clampi(round_i(v[k] * id), -127, 127) & 0xFF) << (8 * k);
        ((uint32_t *)(q80.qs + blk * 256))[lane] = packed;
        if ((lane & 7) == 0) q80.d[blk * 8 + lane / 8] = d;
    }
}

__device__ __forceinline__ float silu_f(float v, float b) { return v / (1.0f + aotk_expf(-v)) * b; }
__device__ __forceinline__ float gelu_f(float v) {
    const float k = (float)1.1283791670955126 / (float)1.4142135623730951;
    return 0.5f * v * (1.0f + aotk_tanhf(k * (v + 0.044715f * v * v * v)));
}


}  // namespace aotk
