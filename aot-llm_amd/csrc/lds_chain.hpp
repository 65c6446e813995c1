// lds_chain.hpp - one thread's in-order f32 sum of a run of LDS values,
// s + p[0] + p[1] + ... , at the latency of the dependent add.
//
// The reads must run well ahead of the adds: an LDS read takes longer than
// several dependent adds. Compiled from plain C++, the reads end up next to
// their use and the chain waits on nearly every one (about 5 ns per element
// on gfx950, against about 3.3 ns here). So the run is written out in
// assembly: 16 values per round, two sets of four 16-byte reads (v96-v111
// and v112-v127, clobbered), the next round's reads issued before the
// current round's adds, and lgkmcnt waits that let exactly those reads stay
// in flight. Every add is a plain v_add_f32 in index order, so the result is
// bit for bit the sequential one.
#pragma once

#include "device.hpp"

namespace aotk {

#define LC_RD(r, off) "ds_read_b128 v[" #r ":" LC_P3(r) "], %[ad] offset:" #off "\n"
#define LC_P3(r) LC_P3_##r
#define LC_P3_96 "99"
#define LC_P3_100 "103"
#define LC_P3_104 "107"
#define LC_P3_108 "111"
#define LC_P3_112 "115"
#define LC_P3_116 "119"
#define LC_P3_120 "123"
#define LC_P3_124 "127"
#define LC_ADD4(a, b, c, d)              \
    "v_add_f32 %[o], %[o], v" #a "\n"    \
    "v_add_f32 %[o], %[o], v" #b "\n"    \
    "v_add_f32 %[o], %[o], v" #c "\n"    \
    "v_add_f32 %[o], %[o], v" #d "\n"
// the current round's 16 values from set A (v96-v111) / set B (v112-v127),
// with W0..W3 the waits before each group of four
#define LC_ADD_A(W0, W1, W2, W3)                                  \
    "s_waitcnt lgkmcnt(" #W0 ")\n" LC_ADD4(96, 97, 98, 99)        \
    "s_waitcnt lgkmcnt(" #W1 ")\n" LC_ADD4(100, 101, 102, 103)    \
    "s_waitcnt lgkmcnt(" #W2 ")\n" LC_ADD4(104, 105, 106, 107)    \
    "s_waitcnt lgkmcnt(" #W3 ")\n" LC_ADD4(108, 109, 110, 111)
#define LC_ADD_B(W0, W1, W2, W3)                                  \
    "s_waitcnt lgkmcnt(" #W0 ")\n" LC_ADD4(112, 113, 114, 115)    \
    "s_waitcnt lgkmcnt(" #W1 ")\n" LC_ADD4(116, 117, 118, 119)    \
    "s_waitcnt lgkmcnt(" #W2 ")\n" LC_ADD4(120, 121, 122, 123)    \
    "s_waitcnt lgkmcnt(" #W3 ")\n" LC_ADD4(124, 125, 126, 127)
// prologue: nothing else outstanding on the counter (it also counts scalar
// loads, which would upset the waits below), then the first round into set A
#define LC_PRO "s_waitcnt lgkmcnt(0)\n" LC_RD(96, 0) LC_RD(100, 16) LC_RD(104, 32) LC_RD(108, 48)
// a round: the next round (64 bytes on) into the other set, the adds of this
// one, then the address moves on
#define LC_RA LC_RD(112, 64) LC_RD(116, 80) LC_RD(120, 96) LC_RD(124, 112) LC_ADD_A(7, 6, 5, 4) "v_add_u32 %[ad], 64, %[ad]\n"
#define LC_RB LC_RD(96, 64) LC_RD(100, 80) LC_RD(104, 96) LC_RD(108, 112) LC_ADD_B(7, 6, 5, 4) "v_add_u32 %[ad], 64, %[ad]\n"
// the last round (in set B): nothing more to read
#define LC_FB LC_ADD_B(3, 2, 1, 0)
#define LC_CLOBBER                                                                                                  \
    "v96", "v97", "v98", "v99", "v100", "v101", "v102", "v103", "v104", "v105", "v106", "v107", "v108", "v109", \
        "v110", "v111", "v112", "v113", "v114", "v115", "v116", "v117", "v118", "v119", "v120", "v121", "v122",  \
        "v123", "v124", "v125", "v126", "v127"

__device__ __forceinline__ uint32_t lds_addr(const float *p) { return (uint32_t)(uintptr_t)p; }

// s + p[0..63] in order (p in LDS, 16-byte aligned).
__device__ __forceinline__ float lds_chain64(const float *p, float s) {
    uint32_t ad = lds_addr(p);
    asm volatile(LC_PRO LC_RA LC_RB LC_RA LC_FB
                 : [o] "+v"(s), [ad] "+v"(ad)
                 :
                 : "memory", LC_CLOBBER);
    return s;
}

// s + p[0..127] in order (p in LDS, 16-byte aligned).
__device__ __forceinline__ float lds_chain128(const float *p, float s) {
    uint32_t ad = lds_addr(p);
    asm volatile(LC_PRO LC_RA LC_RB LC_RA LC_RB LC_RA LC_RB LC_RA LC_FB
                 : [o] "+v"(s), [ad] "+v"(ad)
                 :
                 : "memory", LC_CLOBBER);
    return s;
}

// s + p[0..191] in order (p in LDS, 16-byte aligned).
__device__ __forceinline__ float lds_chain192(const float *p, float s) {
    uint32_t ad = lds_addr(p);
    asm volatile(LC_PRO LC_RA LC_RB LC_RA LC_RB LC_RA LC_RB LC_RA LC_RB LC_RA LC_RB LC_RA LC_FB
                 : [o] "+v"(s), [ad] "+v"(ad)
                 :
                 : "memory", LC_CLOBBER);
    return s;
}

}  // namespace aotk
