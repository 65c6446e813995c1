// seqsum.hpp - exact, parallel replay of a sequential f32 sum of non-negative
// terms: returns bit for bit what `s = 0; for k: s += p[k]` (round to nearest
// even at every step) produces, without an n-long dependent add chain.
//
// The reference sums sequentially (rmsnorm ops.rs:10-13, softmax
// ops.rs:104-107). A wave issues one dependent f32 add per ~4.5 cycles at
// best, so a 4096-term chain is ~8 us; this replay takes a fraction of that.
//
// Method (all terms p_k >= 0, so partial sums never decrease):
//  1. thread t owns the C consecutive elements of chunk t. An f32 block
//     scan of the chunk sums predicts every chunk's range of partial sums.
//     When that range, widened by a margin well above the drift between
//     the true f32 partial sums and the prediction, lies in one binade
//     [2^e, 2^(e+1)), the chunk is a run candidate. The prediction only
//     decides how the work is split; the result never depends on it.
//  2. while the running sum s = A * u (u = 2^(e-23), 2^23 <= A < 2^24) stays
//     in one binade, adding p_k adds round(p_k / u) to the integer A. With
//     no exact .5 fraction that rounding does not depend on s, so a run
//     chunk carries the plain integer sum G of its rounded increments (a
//     chunk holding an exact .5 fraction is not a run). Consecutive run
//     chunks of one binade merge into one event; every other chunk is an
//     event of its own, added element by element.
//  3. one wave walks the events in order: a jump A += G for a run after
//     checking that s lies in the run's binade and that A + G < 2^24 (then,
//     A being monotone, every partial sum of the run did), plain f32 adds
//     otherwise. A failed check adds the run's elements one by one, so the
//     result is the sequential one whatever the prediction said.
// In rows of similar terms the binade changes about log2(n) times, mostly
// early: a 4096-term sum becomes some 20-35 events.
#pragma once

#include "device.hpp"

#ifndef SEQ_TS
#define SEQ_TS(i)
#endif
#ifndef SEQ_STAT
#define SEQ_STAT(k, v)
#endif

namespace aotk {

constexpr int SEQ_MAX_N = 16384;
// The sum runs in blocks of SEQ_T threads, of which the first seq_threads(n)
// own a chunk each (fewer threads carry less fixed per-thread work for short
// sums). The chunk length C = seq_chunk(n) is a power of two. Inputs live in
// LDS in a padded chunk layout: element k of chunk t = k / C is stored at
// t*(C+1) + k % C, so the lanes of a wave walking their chunks spread over
// the banks.
constexpr int SEQ_T = 1024;
constexpr int SEQ_PAD_N = SEQ_MAX_N + SEQ_T + 32;
__device__ __forceinline__ int seq_threads(int n) { return n <= 1024 ? 256 : SEQ_T; }
__device__ __forceinline__ int seq_chunk_of(int n, int t) {  // chunk length for t threads
    const int c = (n + t - 1) / t;
    return c <= 1 ? 1 : 1 << (32 - __builtin_clz(c - 1));
}
__device__ __forceinline__ int seq_chunk(int n) { return seq_chunk_of(n, seq_threads(n)); }
__device__ __forceinline__ int seq_idx(int k, int C) {
    const int lc = __builtin_ctz(C);
    return (k >> lc) * (C + 1) + (k & (C - 1));
}
constexpr int SEQ_SINGLE = -32768;  // code of a chunk added element by element
constexpr int SEQ_NONE = -32767;    // chunk past the end
constexpr int SEQ_G_CAP = 1 << 29;  // merged increments saturate here (a run needs < 2^24)

// Steps in element order: an element step adds p; a run of binade e adds
// G * 2^(e-23), exactly, when the running sum lies in [2^e, 2^(e+1)) and the
// result stays below 2^(e+1). Per step: the value to add (sa, zero past the
// last step), the last element it covers (sz) and
// 2^e for a run, 0 for an element (slo). A run covers the elements after
// the previous step's last one.
constexpr int SEQ_MAX_EV = 2048;
struct __align__(16) SeqScratch {
    float sa[SEQ_MAX_EV + 64];
    float slo[SEQ_MAX_EV];
    int sz[SEQ_MAX_EV];
    int code[SEQ_T];
    float wsum[SEQ_T / 64];
    int wv[SEQ_T / 64], wf[SEQ_T / 64], wc[SEQ_T / 64];
    float result;
};

// Wave-wide inclusive scans with DPP row shifts and row broadcasts (GFX9
// DPP: row_shr 1/2/4/8 within rows of 16 lanes, then row_bcast15 into rows
// 1 and 3, row_bcast31 into rows 2 and 3). Lanes without a source read 0.
template <int CTRL, int ROWS>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROWS, 0xf, true);
}
template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL, ROWS>(__float_as_int(v)));
}
__device__ __forceinline__ float wave_scan_f(float x) {
    x += dpp_f<0x111, 0xf>(x);
    x += dpp_f<0x112, 0xf>(x);
    x += dpp_f<0x114, 0xf>(x);
    x += dpp_f<0x118, 0xf>(x);
    x += dpp_f<0x142, 0xa>(x);
    x += dpp_f<0x143, 0xc>(x);
    return x;
}
// Segmented (v, f) carry plus a plain count c, combined as
// (v1,f1,c1) + (v2,f2,c2) = (f2 ? v2 : min(v1 + v2, cap), f1 | f2, c1 + c2).
template <int CTRL, int ROWS>
__device__ __forceinline__ void seg_step(int &v, int &f, int &c) {
    const int ov = dpp_i<CTRL, ROWS>(v), of = dpp_i<CTRL, ROWS>(f), oc = dpp_i<CTRL, ROWS>(c);
    v = f ? v : min(v + ov, SEQ_G_CAP);
    f |= of;
    c += oc;
}
__device__ __forceinline__ void wave_scan_seg(int &v, int &f, int &c) {
    seg_step<0x111, 0xf>(v, f, c);
    seg_step<0x112, 0xf>(v, f, c);
    seg_step<0x114, 0xf>(v, f, c);
    seg_step<0x118, 0xf>(v, f, c);
    seg_step<0x142, 0xa>(v, f, c);
    seg_step<0x143, 0xc>(v, f, c);
}

__device__ __forceinline__ int flt_exponent(float v) {  // floor(log2(v)) for normal v > 0
    return (int)((__float_as_uint(v) >> 23) & 0xff) - 127;
}

__device__ __forceinline__ float pow2f(int e) { return __int_as_float((127 + e) << 23); }  // -126 <= e <= 127

// Walk of the steps on one wave, 64 at a time. Every lane runs the same
// chain of plain f32 adds over the batch (the values read as LDS
// broadcasts, four per read); lane j recovers the running sum before step
// j; afterwards every lane checks its own run in parallel (s in
// [2^e, 2^(e+1)) and s + G * 2^(e-23) < 2^(e+1): then the add was the exact
// jump A += G). At the first failed check the walk restarts from that step
// and adds the run's elements one by one.
__device__ __forceinline__ float seq_walk(const float *pp, int C, int total, const SeqScratch &S) {
    const int lane = threadIdx.x & 63;
    total = __builtin_amdgcn_readfirstlane(total);
    float s = 0.0f;
    int prev_last = -1;  // last element already added
    int e0 = 0;
    SEQ_TS(6);
    while (e0 < total) {
        // the batch starts at the 16-byte boundary at or below e0; the steps
        // before e0 (done already, after a failed check) add 0 and pass
        const int eb = e0 & ~3, skip = e0 - eb;
        const int cnt = min(64, total - eb);
        float4 av[16];
#pragma unroll
        for (int q = 0; q < 16; q++) av[q] = reinterpret_cast<const float4 *>(S.sa + eb)[q];
        if (skip > 0) {
            av[0].x = 0.0f;
            if (skip > 1) av[0].y = 0.0f;
            if (skip > 2) av[0].z = 0.0f;
        }
        const bool mine = lane >= skip && lane < cnt;
        // this lane's group of four steps (the skipped ones added as 0, as in the chain)
        float4 gv = reinterpret_cast<const float4 *>(S.sa + eb)[lane >> 2];
        if (lane < 4) {
            if (skip > 0) gv.x = 0.0f;
            if (skip > 1) gv.y = 0.0f;
            if (skip > 2) gv.z = 0.0f;
        }
        const float mylo = mine ? S.slo[eb + lane] : 0.0f;
        const int myz = lane < cnt ? S.sz[eb + lane] : 0;
        // the chain keeps the sum before every fourth step in that group's
        // four lanes; each lane then adds its group's steps before its own,
        // in order (the same adds as the chain, so the same roundings)
        float t = s, hist = s;
        const int grp = lane >> 2, r = lane & 3;
        SEQ_TS(7);
#pragma unroll
        for (int q16 = 0; q16 < 4; q16++) {
            if (16 * q16 >= cnt) break;  // (steps past the total add 0)
#pragma unroll
            for (int q = 4 * q16; q < 4 * q16 + 4; q++) {
                hist = grp == q ? t : hist;
                t += av[q].x;
                t += av[q].y;
                t += av[q].z;
                t += av[q].w;
            }
        }
        if (r > 0) hist += gv.x;
        if (r > 1) hist += gv.y;
        if (r > 2) hist += gv.z;
        const float myadd = r == 0 ? gv.x : (r == 1 ? gv.y : (r == 2 ? gv.z : gv.w));
        SEQ_TS(8);
        const bool ok = mylo == 0.0f || (hist >= mylo && hist + myadd < 2.0f * mylo);
        const unsigned long long bad = __ballot(!ok && mine);
        if (bad == 0) {
            s = t;
            prev_last = __builtin_amdgcn_readlane(myz, cnt - 1);
            e0 = eb + cnt;
        } else {
            const int jb = __builtin_ctzll(bad);
            s = readlane_f(hist, jb);
            const int first = (jb == skip ? prev_last : __builtin_amdgcn_readlane(myz, jb - 1)) + 1;
            const int last = __builtin_amdgcn_readlane(myz, jb);
            SEQ_STAT(1, last - first + 1);
            for (int k = first; k <= last; k++) s += pp[seq_idx(k, C)];
            prev_last = last;
            e0 = eb + jb + 1;
        }
    }
    return s;
}

// Exact sequential sum of p[0..n) (LDS, padded layout of seq_idx, all
// p >= 0, 1 <= n <= SEQ_MAX_N). The first T threads own a chunk each
// (T == seq_threads(n), seq_chunk(n) <= MAXC); all threads of the block
// (blockDim.x >= T) call it after p is complete, and all get the result.
template <int MAXC, int T>
__device__ __forceinline__ float exact_seq_sum_t(const float *pp, int n, SeqScratch &S) {
    constexpr int NW = T / 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int C = seq_chunk_of(n, T);
    const bool act = tid < T;  // wave-uniform; idle waves only meet the barriers
    const int c0 = act ? min(tid * C, n) : n;
    const int len = min(c0 + C, n) - c0;
    SEQ_TS(0);
    // 1. chunk sums and their block scan (f32: a prediction only)
    float pr[MAXC];
    float loc = 0.0f, P = 0.0f;
    if (act) {
#pragma unroll
        for (int i = 0; i < MAXC; i++) pr[i] = i < len ? pp[tid * (C + 1) + i] : 0.0f;
#pragma unroll
        for (int i = 0; i < MAXC; i++) loc += pr[i];
        const float incl = wave_scan_f(loc);
        if (lane == 63) S.wsum[wave] = incl;
        P = dpp_f<0x138, 0xf>(incl);  // wave_shr:1, the exclusive prefix within the wave
    }
    __syncthreads();
    SEQ_TS(1);
    // 2. classify the chunk: a run of binade e with increments g, or single
    int code = len > 0 ? SEQ_SINGLE : SEQ_NONE, g = 0;
    if (act) {
        {  // the earlier waves' totals: one read per lane, a scan across lanes
            const float wp = wave_scan_f(lane < NW ? S.wsum[lane] : 0.0f);
            if (wave > 0) P += readlane_f(wp, wave - 1);
        }
        // partial sums of chunk t drift from the prediction by less than
        // (c0 + C + 64) ulp-sized steps of 2^-24 relative
        const float d = (float)(c0 + len + 64) * 0x1p-23f;
        const int elo = flt_exponent(P * (1.0f - d)), ehi = flt_exponent((P + loc) * (1.0f + d));
        if (len > 0 && P > 0.0f && elo == ehi && elo > -100 && elo < 120) {
            const float sc = pow2f(23 - elo);
            bool ok = true;
#pragma unroll
            for (int i = 0; i < MAXC; i++) {
                const float q = pr[i] * sc;  // p / u, exact
                const float fl = floorf(q);
                const float fr = q - fl;
                ok = ok && fr != 0.5f && fl < 16777216.0f;
                g += (int)fl + (fr > 0.5f ? 1 : 0);
            }
            if (ok) code = elo;
            else g = 0;
        }
        S.code[tid] = code;
    }
    __syncthreads();
    SEQ_TS(2);
    // 3. merge consecutive run chunks of one binade; one event per merged run
    //    and per single chunk, numbered by a block scan
    const bool run = code > SEQ_NONE;
    bool cont = false, end = false;
    int v = 0, f = 1, c = 0;
    if (act) {
        const int before = tid > 0 ? S.code[tid - 1] : SEQ_NONE;
        const int after = tid + 1 < T ? S.code[tid + 1] : SEQ_NONE;
        cont = run && before == code;
        end = code != SEQ_NONE && (!run || after != code);
        v = g;
        f = cont ? 0 : 1;
        c = end ? (run ? 1 : len) : 0;
        wave_scan_seg(v, f, c);
        if (lane == 63) {
            S.wv[wave] = v;
            S.wf[wave] = f;
            S.wc[wave] = c;
        }
    }
    __syncthreads();
    SEQ_TS(3);
    int total = 0;
    if (act) {
        // the earlier waves' carries: one read per lane, a scan across lanes
        int lv = lane < NW ? S.wv[lane] : 0, lf = lane < NW ? S.wf[lane] : 1, lc = lane < NW ? S.wc[lane] : 0;
        wave_scan_seg(lv, lf, lc);
        int cv = 0, cc = 0;
        if (wave > 0) {
            cv = __builtin_amdgcn_readlane(lv, wave - 1);
            cc = __builtin_amdgcn_readlane(lc, wave - 1);
        }
        total = __builtin_amdgcn_readlane(lc, NW - 1);
        const int pv = dpp_i<0x138, 0xf>(v), pf = dpp_i<0x138, 0xf>(f), pc = dpp_i<0x138, 0xf>(c);  // wave_shr:1
        cv = pf ? pv : min(cv + pv, SEQ_G_CAP);  // increments of the run's earlier chunks
        cc += pc;                                // steps before this chunk's
        if (end && cc + c <= SEQ_MAX_EV) {
            if (run) {
                // G * 2^(e-23): exact below 2^24; a larger G fails its check anyway
                S.sa[cc] = (float)min((cont ? cv : 0) + g, SEQ_G_CAP) * pow2f(code - 23);
                S.slo[cc] = pow2f(code);
                S.sz[cc] = c0 + len - 1;
            } else {
#pragma unroll
                for (int i = 0; i < MAXC; i++)
                    if (i < len) {
                        S.sa[cc + i] = pr[i];
                        S.slo[cc + i] = 0.0f;
                        S.sz[cc + i] = c0 + i;
                    }
            }
        }
        if (tid < 64) S.sa[min(total, SEQ_MAX_EV) + tid] = 0.0f;  // the last batch's padding
    }
    __syncthreads();
    SEQ_TS(4);
    // 4. walk on wave 0 (past SEQ_MAX_EV steps, element by element; wave 0
    //    always owns chunks and knows the total)
    if (wave == 0) {
        SEQ_STAT(0, total);
        float s = 0.0f;
        if (total <= SEQ_MAX_EV) {
            s = seq_walk(pp, C, total, S);
        } else {
            for (int k = 0; k < n; k++) s += pp[seq_idx(k, C)];
        }
        if (lane == 0) S.result = s;
    }
    __syncthreads();
    SEQ_TS(5);
    return S.result;
}

// The same sum on a block of 256 threads (n <= 8192; the inputs in the
// layout of seq_idx with C = seq_chunk_of(n, 256)): about twice the latency
// of the 1024-thread form, half its instructions, for kernels that run many
// independent sums at once.
__device__ __forceinline__ float exact_seq_sum256(const float *pp, int n, SeqScratch &S) {
    const int C = seq_chunk_of(n, 256);
    if (C <= 4) return exact_seq_sum_t<4, 256>(pp, n, S);
    if (C <= 8) return exact_seq_sum_t<8, 256>(pp, n, S);
    if (C <= 16) return exact_seq_sum_t<16, 256>(pp, n, S);
    return exact_seq_sum_t<32, 256>(pp, n, S);
}

__device__ __forceinline__ float exact_seq_sum(const float *pp, int n, SeqScratch &S) {
    if (seq_threads(n) == 256) return exact_seq_sum_t<4, 256>(pp, n, S);
    if (seq_chunk(n) <= 4) return exact_seq_sum_t<4, SEQ_T>(pp, n, S);
    if (seq_chunk(n) <= 8) return exact_seq_sum_t<8, SEQ_T>(pp, n, S);
    return exact_seq_sum_t<SEQ_MAX_N / SEQ_T, SEQ_T>(pp, n, S);
}

}  // namespace aotk
