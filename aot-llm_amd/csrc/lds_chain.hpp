// lds_chain.hpp - one thread's in-order f32 sum of a run of LDS values,
// s + p[0] + p[1] + ... , at close to the issue rate of the dependent add.
//
// A wave issues about one instruction per 4.5 cycles, and a dependent
// v_add_f32 needs no more, so the run costs the adds plus whatever else the
// wave issues. The LDS reads must also run well ahead of the adds: a read
// takes longer than many dependent adds, more so while other waves write
// LDS. Compiled from plain C++, the reads end up next to their use and the
// chain waits on nearly every one. So the run is written out in assembly:
// groups of four values, each read by one ds_read_b128 with an immediate
// offset (no address arithmetic), into eight register sets v96-v127
// (clobbered) in turn; the read of group g + 7 is issued before the adds of
// group g, after a single lgkmcnt wait that lets the seven younger reads stay
// in flight. Every add is a plain v_add_f32 in index order, so the result is
// bit for bit the sequential one.
#pragma once

#include "device.hpp"

namespace aotk {

#define LC_W(n) "s_waitcnt lgkmcnt(" #n ")\n"
#define LC_RD(lo, hi, off) "ds_read_b128 v[" #lo ":" #hi "], %[ad] offset:" #off "\n"
#define LC_R0(off) LC_RD(96, 99, off)
#define LC_R1(off) LC_RD(100, 103, off)
#define LC_R2(off) LC_RD(104, 107, off)
#define LC_R3(off) LC_RD(108, 111, off)
#define LC_R4(off) LC_RD(112, 115, off)
#define LC_R5(off) LC_RD(116, 119, off)
#define LC_R6(off) LC_RD(120, 123, off)
#define LC_R7(off) LC_RD(124, 127, off)
#define LC_ADD4(a, b, c, d)              \
    "v_add_f32 %[o], %[o], v" #a "\n"    \
    "v_add_f32 %[o], %[o], v" #b "\n"    \
    "v_add_f32 %[o], %[o], v" #c "\n"    \
    "v_add_f32 %[o], %[o], v" #d "\n"
#define LC_A0 LC_ADD4(96, 97, 98, 99)
#define LC_A1 LC_ADD4(100, 101, 102, 103)
#define LC_A2 LC_ADD4(104, 105, 106, 107)
#define LC_A3 LC_ADD4(108, 109, 110, 111)
#define LC_A4 LC_ADD4(112, 113, 114, 115)
#define LC_A5 LC_ADD4(116, 117, 118, 119)
#define LC_A6 LC_ADD4(120, 121, 122, 123)
#define LC_A7 LC_ADD4(124, 125, 126, 127)
// (the first wait also drains anything else outstanding on the counter,
// which counts scalar loads too and would upset the waits that follow)
#define LC_CLOBBER                                                                                                  \
    "v96", "v97", "v98", "v99", "v100", "v101", "v102", "v103", "v104", "v105", "v106", "v107", "v108", "v109", \
        "v110", "v111", "v112", "v113", "v114", "v115", "v116", "v117", "v118", "v119", "v120", "v121", "v122",  \
        "v123", "v124", "v125", "v126", "v127"

__device__ __forceinline__ uint32_t lds_addr(const float *p) { return (uint32_t)(uintptr_t)p; }

// s + p[0..63] in order (p in LDS, 16-byte aligned).
__device__ __forceinline__ float lds_chain64(const float *p, float s) {
    const uint32_t ad = lds_addr(p);
    asm volatile(
        LC_W(0)
        LC_R0(0)
        LC_R1(16)
        LC_R2(32)
        LC_R3(48)
        LC_R4(64)
        LC_R5(80)
        LC_R6(96)
        LC_R7(112) LC_W(7) LC_A0
        LC_R0(128) LC_W(7) LC_A1
        LC_R1(144) LC_W(7) LC_A2
        LC_R2(160) LC_W(7) LC_A3
        LC_R3(176) LC_W(7) LC_A4
        LC_R4(192) LC_W(7) LC_A5
        LC_R5(208) LC_W(7) LC_A6
        LC_R6(224) LC_W(7) LC_A7
        LC_R7(240) LC_W(7) LC_A0
        LC_W(6) LC_A1
        LC_W(5) LC_A2
        LC_W(4) LC_A3
        LC_W(3) LC_A4
        LC_W(2) LC_A5
        LC_W(1) LC_A6
        LC_W(0) LC_A7
        : [o] "+v"(s)
        : [ad] "v"(ad)
        : "memory", LC_CLOBBER);
    return s;
}

// s + p[0..127] in order (p in LDS, 16-byte aligned).
__device__ __forceinline__ float lds_chain128(const float *p, float s) {
    const uint32_t ad = lds_addr(p);
    asm volatile(
        LC_W(0)
        LC_R0(0)
        LC_R1(16)
        LC_R2(32)
        LC_R3(48)
        LC_R4(64)
        LC_R5(80)
        LC_R6(96)
        LC_R7(112) LC_W(7) LC_A0
        LC_R0(128) LC_W(7) LC_A1
        LC_R1(144) LC_W(7) LC_A2
        LC_R2(160) LC_W(7) LC_A3
        LC_R3(176) LC_W(7) LC_A4
        LC_R4(192) LC_W(7) LC_A5
        LC_R5(208) LC_W(7) LC_A6
        LC_R6(224) LC_W(7) LC_A7
        LC_R7(240) LC_W(7) LC_A0
        LC_R0(256) LC_W(7) LC_A1
        LC_R1(272) LC_W(7) LC_A2
        LC_R2(288) LC_W(7) LC_A3
        LC_R3(304) LC_W(7) LC_A4
        LC_R4(320) LC_W(7) LC_A5
        LC_R5(336) LC_W(7) LC_A6
        LC_R6(352) LC_W(7) LC_A7
        LC_R7(368) LC_W(7) LC_A0
        LC_R0(384) LC_W(7) LC_A1
        LC_R1(400) LC_W(7) LC_A2
        LC_R2(416) LC_W(7) LC_A3
        LC_R3(432) LC_W(7) LC_A4
        LC_R4(448) LC_W(7) LC_A5
        LC_R5(464) LC_W(7) LC_A6
        LC_R6(480) LC_W(7) LC_A7
        LC_R7(496) LC_W(7) LC_A0
        LC_W(6) LC_A1
        LC_W(5) LC_A2
        LC_W(4) LC_A3
        LC_W(3) LC_A4
        LC_W(2) LC_A5
        LC_W(1) LC_A6
        LC_W(0) LC_A7
        : [o] "+v"(s)
        : [ad] "v"(ad)
        : "memory", LC_CLOBBER);
    return s;
}

// s + p[0..191] in order (p in LDS, 16-byte aligned).
__device__ __forceinline__ float lds_chain192(const float *p, float s) {
    const uint32_t ad = lds_addr(p);
    asm volatile(
        LC_W(0)
        LC_R0(0)
        LC_R1(16)
        LC_R2(32)
        LC_R3(48)
        LC_R4(64)
        LC_R5(80)
        LC_R6(96)
        LC_R7(112) LC_W(7) LC_A0
        LC_R0(128) LC_W(7) LC_A1
        LC_R1(144) LC_W(7) LC_A2
        LC_R2(160) LC_W(7) LC_A3
        LC_R3(176) LC_W(7) LC_A4
        LC_R4(192) LC_W(7) LC_A5
        LC_R5(208) LC_W(7) LC_A6
        LC_R6(224) LC_W(7) LC_A7
        LC_R7(240) LC_W(7) LC_A0
        LC_R0(256) LC_W(7) LC_A1
        LC_R1(272) LC_W(7) LC_A2
        LC_R2(288) LC_W(7) LC_A3
        LC_R3(304) LC_W(7) LC_A4
        LC_R4(320) LC_W(7) LC_A5
        LC_R5(336) LC_W(7) LC_A6
        LC_R6(352) LC_W(7) LC_A7
        LC_R7(368) LC_W(7) LC_A0
        LC_R0(384) LC_W(7) LC_A1
        LC_R1(400) LC_W(7) LC_A2
        LC_R2(416) LC_W(7) LC_A3
        LC_R3(432) LC_W(7) LC_A4
        LC_R4(448) LC_W(7) LC_A5
        LC_R5(464) LC_W(7) LC_A6
        LC_R6(480) LC_W(7) LC_A7
        LC_R7(496) LC_W(7) LC_A0
        LC_R0(512) LC_W(7) LC_A1
        LC_R1(528) LC_W(7) LC_A2
        LC_R2(544) LC_W(7) LC_A3
        LC_R3(560) LC_W(7) LC_A4
        LC_R4(576) LC_W(7) LC_A5
        LC_R5(592) LC_W(7) LC_A6
        LC_R6(608) LC_W(7) LC_A7
        LC_R7(624) LC_W(7) LC_A0
        LC_R0(640) LC_W(7) LC_A1
        LC_R1(656) LC_W(7) LC_A2
        LC_R2(672) LC_W(7) LC_A3
        LC_R3(688) LC_W(7) LC_A4
        LC_R4(704) LC_W(7) LC_A5
        LC_R5(720) LC_W(7) LC_A6
        LC_R6(736) LC_W(7) LC_A7
        LC_R7(752) LC_W(7) LC_A0
        LC_W(6) LC_A1
        LC_W(5) LC_A2
        LC_W(4) LC_A3
        LC_W(3) LC_A4
        LC_W(2) LC_A5
        LC_W(1) LC_A6
        LC_W(0) LC_A7
        : [o] "+v"(s)
        : [ad] "v"(ad)
        : "memory", LC_CLOBBER);
    return s;
}

}  // namespace aotk
