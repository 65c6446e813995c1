// device.hpp - bit-exact scalar helpers for gfx950 device code.
// Every translation unit is compiled with -ffp-contract=off so a*b+c stays two
// roundings unless fmaf() is written explicitly (the reference's Rust never
// contracts outside its FMA intrinsics).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace aotk {

// IEEE binary16 -> f32 (crates/aot-kernels/src/quant.rs:96-125). Zeros,
// subnormals and normals convert exactly in hardware (v_cvt_f32_f16, f16
// denormals on); infinities and NaNs take the integer form so that NaN
// payloads match the reference bit for bit (the hardware quiets them).
__device__ __forceinline__ float f16_to_f32(uint32_t h) {
    const float hw = (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
    const uint32_t special = ((h & 0x8000u) << 16) | 0x7F800000u | ((h & 0x3FFu) << 13);
    // all ones for exponent 31 (Inf / NaN), else zero: a mask, not a
    // compare, so that no branch (and no early wait for a loaded h) forms
    const uint32_t m = 0u - ((((h & 0x7C00u) + 0x400u) >> 15) & 1u);
    return __uint_as_float((special & m) | (__float_as_uint(hw) & ~m));
}

// f32 -> binary16, round to nearest even (quant.rs:128-162).
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    uint32_t x = __float_as_uint(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    int32_t exp = (int32_t)((x >> 23) & 0xFFu);
    uint32_t mant = x & 0x7FFFFFu;
    if (exp == 0xFF) return sign | 0x7C00u | (mant != 0 ? 0x200u : 0u);
    exp -= 127;
    if (exp > 15) return sign | 0x7C00u;
    if (exp < -25) return sign;
    if (exp < -14) {
        uint32_t m = mant | 0x800000u;
        uint32_t shift = (uint32_t)(-14 - exp) + 13;
        uint32_t half = 1u << (shift - 1);
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t r = m >> shift;
        if (rem > half || (rem == half && (r & 1u) == 1u)) r += 1;
        return sign | (uint16_t)r;
    }
    uint32_t r = ((uint32_t)(exp + 15) << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u) == 1u)) r += 1;
    return sign | (uint16_t)r;
}

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t x = __float_as_uint(f);
    if ((x & 0x7F800000u) == 0x7F800000u) return (uint16_t)((x >> 16) | ((x & 0x7FFFFFu) != 0 ? 0x40u : 0u));
    uint32_t lsb = (x >> 16) & 1u;
    return (uint16_t)((x + 0x7FFFu + lsb) >> 16);
}

// Rust `x.round() as i32`: half away from zero, saturating, NaN -> 0.
__device__ __forceinline__ int32_t round_i(float x) {
    float r = roundf(x);
    if (r != r) return 0;
    if (r >= 2147483648.0f) return 2147483647;
    if (r < -2147483648.0f) return (int32_t)0x80000000u;
    return (int32_t)r;
}

__device__ __forceinline__ int32_t clampi(int32_t v, int32_t lo, int32_t hi) { return v < lo ? lo : (v > hi ? hi : v); }

// get_scale_min_k4 (quant.rs:292-298) on the 12 packed scale bytes held in
// three little-endian words.
__device__ __forceinline__ void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2, int &sc, int &m) {
    auto byte = [&](int i) -> uint32_t {
        uint32_t w = i < 4 ? s0 : (i < 8 ? s1 : s2);
        return (w >> (8 * (i & 3))) & 0xFFu;
    };
    if (j < 4) {
        sc = (int)(byte(j) & 63u);
        m = (int)(byte(j + 4) & 63u);
    } else {
        sc = (int)((byte(j + 4) & 0xFu) | ((byte(j - 4) >> 6) << 4));
        m = (int)((byte(j + 4) >> 4) | ((byte(j) >> 6) << 4));
    }
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) { return __builtin_amdgcn_sdot4((int)a, (int)b, c, false); }

// Orders this wave's LDS accesses only (a full fence would also wait for
// outstanding global stores).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int mask) {
    return __shfl_xor(v, mask, 64);
}

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

// Synthetic weight generator (same definition as the oracle's): a sum of four
// uniform 16-bit integers scaled to standard deviation 0.02, exact in f32 up
// to one rounding, so host and device produce identical values.
#define AOTK_SYNTH_SCALE 0x1.1bc77ap-21f
__device__ __forceinline__ float synth_value(uint64_t seed, uint32_t tensor_index, uint64_t elem) {
    uint64_t key = (seed * 0x9E3779B97F4A7C15ULL) ^ ((uint64_t)(tensor_index + 1) << 40) ^ elem;
    uint64_t z = mix64(key);
    int32_t s = (int32_t)(z & 0xFFFF) + (int32_t)((z >> 16) & 0xFFFF) + (int32_t)((z >> 32) & 0xFFFF) +
                (int32_t)(z >> 48) - 131070;
    return (float)s * AOTK_SYNTH_SCALE;
}

}  // namespace aotk

#include "libm_match.h"
#include "libm_tables.h"

namespace aotk {

__device__ __constant__ static const uint32_t expf_exc[][2] = {AOTK_EXPF_EXC_DATA};
__device__ __constant__ static const uint32_t tanhf_exc[][2] = {AOTK_TANHF_EXC_DATA};

__device__ __forceinline__ bool exc_lookup(const uint32_t (*tab)[2], int n, uint32_t key, uint32_t &out) {
    int lo = 0, hi = n;
    while (lo < hi) {
        int mid = (lo + hi) >> 1;
        if (tab[mid][0] < key) lo = mid + 1;
        else hi = mid;
    }
    if (lo < n && tab[lo][0] == key) {
        out = tab[lo][1];
        return true;
    }
    return false;
}

// expf / tanhf bit-identical to the host libm the reference links against.
// aotk_expf_tab reads the 2^(i/32) table from a copy (exp_table_to_lds: in
// LDS a lookup costs an LDS read instead of a constant-memory load).
__device__ __forceinline__ float aotk_expf_tab(float x, const uint64_t *tab) {
    uint32_t o;
    if (AOTK_EXPF_EXC_N && exc_lookup(expf_exc, AOTK_EXPF_EXC_N, __float_as_uint(x), o)) return __uint_as_float(o);
    return lm_expf_tab(x, tab);
}
__device__ __forceinline__ float aotk_expf(float x) { return aotk_expf_tab(x, lm_exp2f_tab_dev); }
// The first 32 threads copy the table (the caller synchronises before use).
__device__ __forceinline__ void exp_table_to_lds(uint64_t *dst) {
    if (threadIdx.x < 32) dst[threadIdx.x] = lm_exp2f_tab_dev[threadIdx.x];
}
__device__ __forceinline__ float aotk_tanhf(float x) {
    uint32_t o;
    if (AOTK_TANHF_EXC_N && exc_lookup(tanhf_exc, AOTK_TANHF_EXC_N, __float_as_uint(x), o)) return __uint_as_float(o);
    return lm_tanhf(x);
}

}  // namespace aotk
