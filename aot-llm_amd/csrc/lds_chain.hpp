// lds_chain.hpp - one thread's in-order f32 sum of a run of LDS values,
// s + p[0] + p[1] + ... , at close to the issue rate of the wave.
//
// A wave issues about one instruction per 4.5 cycles and a dependent
// v_add_f32 needs no more, so the run costs the adds plus whatever else the
// wave issues: the LDS reads (one ds_read_b128 per four values) and the
// waits. Compiled from plain C++, the reads end up next to their use and the
// chain waits on nearly every one. So the run is written out in assembly:
// two sets of sixteen registers, v96-v111 and v112-v127 (clobbered); the
// four reads of the next set (immediate offsets, no address arithmetic) go
// out before the sixteen adds of the current one, after a single lgkmcnt
// wait for the current set. Measured alone on gfx950 this runs at about
// 6.8 cycles per value (7.5 with a wait per four values). Every add is a
// plain v_add_f32 in index order, so the result is bit for bit the
// sequential one.
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
        LC_W(0) LC_R0(0) LC_R1(16) LC_R2(32) LC_R3(48)
        LC_R4(64) LC_R5(80) LC_R6(96) LC_R7(112) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(128) LC_R1(144) LC_R2(160) LC_R3(176) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(192) LC_R5(208) LC_R6(224) LC_R7(240) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_W(0) LC_A4 LC_A5 LC_A6 LC_A7
        : [o] "+v"(s)
        : [ad] "v"(ad)
        : "memory", LC_CLOBBER);
    return s;
}

// s + p[0..127] in order (p in LDS, 16-byte aligned).
__device__ __forceinline__ float lds_chain128(const float *p, float s) {
    const uint32_t ad = lds_addr(p);
    asm volatile(
        LC_W(0) LC_R0(0) LC_R1(16) LC_R2(32) LC_R3(48)
        LC_R4(64) LC_R5(80) LC_R6(96) LC_R7(112) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(128) LC_R1(144) LC_R2(160) LC_R3(176) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(192) LC_R5(208) LC_R6(224) LC_R7(240) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(256) LC_R1(272) LC_R2(288) LC_R3(304) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(320) LC_R5(336) LC_R6(352) LC_R7(368) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(384) LC_R1(400) LC_R2(416) LC_R3(432) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(448) LC_R5(464) LC_R6(480) LC_R7(496) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_W(0) LC_A4 LC_A5 LC_A6 LC_A7
        : [o] "+v"(s)
        : [ad] "v"(ad)
        : "memory", LC_CLOBBER);
    return s;
}

// s + p[0..191] in order (p in LDS, 16-byte aligned).
__device__ __forceinline__ float lds_chain192(const float *p, float s) {
    const uint32_t ad = lds_addr(p);
    asm volatile(
        LC_W(0) LC_R0(0) LC_R1(16) LC_R2(32) LC_R3(48)
        LC_R4(64) LC_R5(80) LC_R6(96) LC_R7(112) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(128) LC_R1(144) LC_R2(160) LC_R3(176) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(192) LC_R5(208) LC_R6(224) LC_R7(240) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(256) LC_R1(272) LC_R2(288) LC_R3(304) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(320) LC_R5(336) LC_R6(352) LC_R7(368) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(384) LC_R1(400) LC_R2(416) LC_R3(432) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(448) LC_R5(464) LC_R6(480) LC_R7(496) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(512) LC_R1(528) LC_R2(544) LC_R3(560) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(576) LC_R5(592) LC_R6(608) LC_R7(624) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(640) LC_R1(656) LC_R2(672) LC_R3(688) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(704) LC_R5(720) LC_R6(736) LC_R7(752) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_W(0) LC_A4 LC_A5 LC_A6 LC_A7
        : [o] "+v"(s)
        : [ad] "v"(ad)
        : "memory", LC_CLOBBER);
    return s;
}

// s + p[0..255] in order (p in LDS, 16-byte aligned).
__device__ __forceinline__ float lds_chain256(const float *p, float s) {
    const uint32_t ad = lds_addr(p);
    asm volatile(
        LC_W(0) LC_R0(0) LC_R1(16) LC_R2(32) LC_R3(48)
        LC_R4(64) LC_R5(80) LC_R6(96) LC_R7(112) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(128) LC_R1(144) LC_R2(160) LC_R3(176) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(192) LC_R5(208) LC_R6(224) LC_R7(240) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(256) LC_R1(272) LC_R2(288) LC_R3(304) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(320) LC_R5(336) LC_R6(352) LC_R7(368) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(384) LC_R1(400) LC_R2(416) LC_R3(432) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(448) LC_R5(464) LC_R6(480) LC_R7(496) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(512) LC_R1(528) LC_R2(544) LC_R3(560) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(576) LC_R5(592) LC_R6(608) LC_R7(624) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(640) LC_R1(656) LC_R2(672) LC_R3(688) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(704) LC_R5(720) LC_R6(736) LC_R7(752) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(768) LC_R1(784) LC_R2(800) LC_R3(816) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(832) LC_R5(848) LC_R6(864) LC_R7(880) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(896) LC_R1(912) LC_R2(928) LC_R3(944) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(960) LC_R5(976) LC_R6(992) LC_R7(1008) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_W(0) LC_A4 LC_A5 LC_A6 LC_A7
        : [o] "+v"(s)
        : [ad] "v"(ad)
        : "memory", LC_CLOBBER);
    return s;
}

// s + p[0..383] in order (p in LDS, 16-byte aligned).
__device__ __forceinline__ float lds_chain384(const float *p, float s) {
    const uint32_t ad = lds_addr(p);
    asm volatile(
        LC_W(0) LC_R0(0) LC_R1(16) LC_R2(32) LC_R3(48)
        LC_R4(64) LC_R5(80) LC_R6(96) LC_R7(112) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(128) LC_R1(144) LC_R2(160) LC_R3(176) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(192) LC_R5(208) LC_R6(224) LC_R7(240) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(256) LC_R1(272) LC_R2(288) LC_R3(304) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(320) LC_R5(336) LC_R6(352) LC_R7(368) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(384) LC_R1(400) LC_R2(416) LC_R3(432) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(448) LC_R5(464) LC_R6(480) LC_R7(496) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(512) LC_R1(528) LC_R2(544) LC_R3(560) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(576) LC_R5(592) LC_R6(608) LC_R7(624) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(640) LC_R1(656) LC_R2(672) LC_R3(688) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(704) LC_R5(720) LC_R6(736) LC_R7(752) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(768) LC_R1(784) LC_R2(800) LC_R3(816) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(832) LC_R5(848) LC_R6(864) LC_R7(880) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(896) LC_R1(912) LC_R2(928) LC_R3(944) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(960) LC_R5(976) LC_R6(992) LC_R7(1008) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(1024) LC_R1(1040) LC_R2(1056) LC_R3(1072) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(1088) LC_R5(1104) LC_R6(1120) LC_R7(1136) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(1152) LC_R1(1168) LC_R2(1184) LC_R3(1200) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(1216) LC_R5(1232) LC_R6(1248) LC_R7(1264) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(1280) LC_R1(1296) LC_R2(1312) LC_R3(1328) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(1344) LC_R5(1360) LC_R6(1376) LC_R7(1392) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_R0(1408) LC_R1(1424) LC_R2(1440) LC_R3(1456) LC_W(4) LC_A4 LC_A5 LC_A6 LC_A7
        LC_R4(1472) LC_R5(1488) LC_R6(1504) LC_R7(1520) LC_W(4) LC_A0 LC_A1 LC_A2 LC_A3
        LC_W(0) LC_A4 LC_A5 LC_A6 LC_A7
        : [o] "+v"(s)
        : [ad] "v"(ad)
        : "memory", LC_CLOBBER);
    return s;
}

}  // namespace aotk
