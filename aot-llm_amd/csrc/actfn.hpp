// actfn.hpp - device helpers shared by the matvec and the ops kernels: the
// activation quantizers of one 256-value block held by a wave, and the GLU
// activations.
#pragma once

#include "device.hpp"
#include "internal.hpp"

namespace aotk {

// Quantize 256 values held 4 per lane (element 4*lane + k) of one wave into
// the Q8_K block `blk` (quant.rs:248-283) and/or the 8 Q8_0 blocks
// 8*blk .. 8*blk+7 (quant.rs:231-245).
__device__ __forceinline__ void quant256(const float v[4], int lane, size_t blk, ActQ8K q8k, ActQ8_0 q80) {
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

__device__ __forceinline__ float silu_f(float v, float b) { return v / (1.0f + aotk_expf(-v)) * b; }
__device__ __forceinline__ float gelu_f(float v) {
    const float k = (float)1.1283791670955126 / (float)1.4142135623730951;
    return 0.5f * v * (1.0f + aotk_tanhf(k * (v + 0.044715f * v * v * v)));
}


}  // namespace aotk
