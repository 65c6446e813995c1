// seqsum.hpp - exact, parallel replay of a sequential f32 sum of non-negative
// terms: returns bit for bit what `s = 0; for k: s += p[k]` (round to nearest
// even at every step) produces, without an n-long dependent add chain.
//
// The reference sums sequentially (rmsnorm ops.rs:10-13, softmax
// ops.rs:104-107). A dependent f32 add costs ~3 ns on gfx950, so a 4096-term
// chain is ~13 us; this replay takes a few.
//
// Method (all terms p_k >= 0, so partial sums never decrease):
//  1. prefix sums P_k in double predict each partial sum s_k; s_k differs
//     from P_k by at most k * 2^-24 * s_k, so a predicted binade
//     [2^e, 2^(e+1)) shared by P_(k-1) and P_k with that margin is almost
//     always the true one. The prediction only decides how the work is
//     split; the result never depends on it (step 3 checks every jump).
//  2. while the running sum s = A * u (u = 2^(e-23), 2^23 <= A < 2^24) stays
//     in one binade, adding p_k adds round(p_k / u) to the integer A. With
//     no exact .5 fraction that rounding is unambiguous, so a run of such
//     elements adds the plain integer sum of its increments. Elements whose
//     binade is uncertain, or whose p_k / u ends in exactly .5, are single
//     events (one real f32 add each).
//  3. one wave walks the compacted events in order: an add for a single
//     element, a jump A += G for a run after checking that s lies in the
//     run's binade and that A + G < 2^24 (then, A being monotone, every
//     partial sum of the run did). A failed check adds the run's elements
//     one by one, so the result is the sequential one whatever happened.
#pragma once

#include "device.hpp"

#ifndef SEQ_TS
#define SEQ_TS(i)
#endif

namespace aotk {

constexpr int SEQ_MAX_N = 8192;
// The sum runs in blocks of SEQ_T threads, of which the first seq_threads(n)
// do the work (fewer threads carry less fixed per-thread work for short
// sums). Inputs live in LDS in a padded chunk layout: working thread t owns
// elements [t*C, t*C+C) (C = seq_chunk(n)) stored at t*(C+1) + i, so the
// lanes of a wave walking their chunks spread over the banks.
constexpr int SEQ_T = 1024;
constexpr int SEQ_PAD_N = SEQ_MAX_N + SEQ_T + 32;
constexpr int SEQ_MID_N = 4096;  // sums up to this length run on 512 threads
__device__ __forceinline__ int seq_threads(int n) { return n <= 1024 ? 256 : (n <= SEQ_MID_N ? 512 : SEQ_T); }
__device__ __forceinline__ int seq_chunk(int n) { return (n + seq_threads(n) - 1) / seq_threads(n); }
__device__ __forceinline__ int seq_idx(int k, int C) { return (k / C) * (C + 1) + (k % C); }
constexpr int SEQ_MAX_EV = 2048;
constexpr int SEQ_SINGLE = -32768;  // binade code of an element added alone

// Events are stored in order, each at the slot of its last element: a
// single element (e == SEQ_SINGLE) or a run of elements of binade e whose
// rounded increments sum to g.
struct SeqScratch {
    int4 ev[SEQ_MAX_EV];  // {last element, e, g, 0}
    int e_first[SEQ_T], e_last[SEQ_T];
    int wv[SEQ_T / 64], wf[SEQ_T / 64], wc[SEQ_T / 64];
    double wd[SEQ_T / 64];
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
__device__ __forceinline__ double dpp_d(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = dpp_i<CTRL, ROWS>((int)(b & 0xffffffffLL)), hi = dpp_i<CTRL, ROWS>((int)(b >> 32));
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}
__device__ __forceinline__ double wave_scan_d(double x) {
    x += dpp_d<0x111, 0xf>(x);
    x += dpp_d<0x112, 0xf>(x);
    x += dpp_d<0x114, 0xf>(x);
    x += dpp_d<0x118, 0xf>(x);
    x += dpp_d<0x142, 0xa>(x);
    x += dpp_d<0x143, 0xc>(x);
    return x;
}
// Segmented (v, f) carry plus a plain count c, combined as
// (v1,f1,c1) + (v2,f2,c2) = (f2 ? v2 : v1 + v2, f1 | f2, c1 + c2).
template <int CTRL, int ROWS>
__device__ __forceinline__ void seg_step(int &v, int &f, int &c) {
    const int ov = dpp_i<CTRL, ROWS>(v), of = dpp_i<CTRL, ROWS>(f), oc = dpp_i<CTRL, ROWS>(c);
    v = f ? v : v + ov;
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

__device__ __forceinline__ int dbl_exponent(double v) {  // floor(log2(v)) for normal v > 0
    return (int)((__double_as_longlong(v) >> 52) & 0x7ff) - 1023;
}

__device__ __forceinline__ float pow2f(int e) { return __int_as_float((127 + e) << 23); }  // -126 <= e <= 127

// Walk of the events on one wave. Each lane holds one event of a batch of
// 64 as an affine step s -> fma(s, sc, add) * inv: (1, p, 1) for a single
// element (the f32 add itself), (2^(23-e), G, 2^(e-23)) for a run (exact:
// s * 2^(23-e) is the integer significand A). The chain runs unchecked; the
// running sum before every event is kept in lane j of `hist`, and afterwards
// every lane checks its own run in parallel (s in [2^e, 2^(e+1)) and
// A + G < 2^24). At the first failed check the walk restarts from that
// event and adds its elements one by one.
template <int MAXC>
__device__ __forceinline__ float seq_walk(const float *pp, int C, int total, const SeqScratch &S) {
    const int lane = threadIdx.x & 63;
    float s = 0.0f;
    int prev_last = -1;  // last element already added
    int e0 = 0;
    while (e0 < total) {
        const int cnt = min(64, total - e0);
        int4 E = make_int4(-1, SEQ_SINGLE, 0, 0);
        if (lane < cnt) E = S.ev[e0 + lane];
        const bool run = E.y != SEQ_SINGLE;
        const int e = run ? E.y : 0;
        const float sc = run ? pow2f(23 - e) : 1.0f;
        const float inv = run ? pow2f(e - 23) : 1.0f;
        const float add = run ? (float)E.z : (lane < cnt ? pp[seq_idx(E.x, C)] : 0.0f);
        float t = s, hist = s;
#pragma unroll
        for (int j0 = 0; j0 < 64; j0 += 16) {
            if (j0 >= cnt) break;
#pragma unroll
            for (int j = j0; j < j0 + 16; j++) {
                hist = lane == j ? t : hist;
                const float scj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sc), j));
                const float addj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(add), j));
                const float invj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv), j));
                t = __builtin_fmaf(t, scj, addj) * invj;
            }
        }
        const float lo = pow2f(e);
        const bool ok = !run || (hist >= lo && hist < 2.0f * lo && __builtin_fmaf(hist, sc, add) < 16777216.0f);
        const unsigned long long bad = __ballot(!ok && lane < cnt);
        if (bad == 0) {
            s = t;
            prev_last = __builtin_amdgcn_readlane(E.x, cnt - 1);
            e0 += cnt;
        } else {
            const int jb = __builtin_ctzll(bad);
            s = readlane_f(hist, jb);
            const int first = (jb == 0 ? prev_last : __builtin_amdgcn_readlane(E.x, jb - 1)) + 1;
            const int last = __builtin_amdgcn_readlane(E.x, jb);
            for (int k = first; k <= last; k++) s += pp[seq_idx(k, C)];
            prev_last = last;
            e0 += jb + 1;
        }
    }
    return s;
}

// Exact sequential sum of p[0..n) (LDS, padded layout of seq_idx, all
// p >= 0, 1 <= n <= SEQ_MAX_N). The first T threads work (T == seq_threads(n),
// seq_chunk(n) <= MAXC); all SEQ_T threads of the block call it after p is
// complete, and all get the result.
template <int MAXC, int T>
__device__ __forceinline__ float exact_seq_sum_t(const float *pp, int n, SeqScratch &S) {
    constexpr int NW = T / 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int C = seq_chunk(n);
    const bool act = tid < T;  // wave-uniform; idle waves only meet the barriers
    const int c0 = act ? min(tid * C, n) : n, c1 = min(c0 + C, n);
    const int len = c1 - c0;
    const int base = tid * (C + 1);
    SEQ_TS(0);
    // 1. double prefix sums
    float pr[MAXC];
    double loc = 0.0, P = 0.0;
    if (act) {
#pragma unroll
        for (int i = 0; i < MAXC; i++) pr[i] = i < len ? pp[base + i] : 0.0f;
#pragma unroll
        for (int i = 0; i < MAXC; i++) loc += (double)pr[i];
        const double incl = wave_scan_d(loc);
        if (lane == 63) S.wd[wave] = incl;
        P = incl - loc;
    }
    __syncthreads();
    if (act) {
#pragma unroll
        for (int w = 0; w < NW - 1; w++)
            if (w < wave) P += S.wd[w];
    }
    SEQ_TS(1);
    // 2. classify: binade code and rounded increment of each element. The
    //    margin (c1 + 2) * 2^-23 bounds the drift of every partial sum of
    //    the chunk.
    int ec[MAXC], g[MAXC];
#pragma unroll
    for (int i = 0; i < MAXC; i++) {
        ec[i] = SEQ_SINGLE;
        g[i] = 0;
    }
    int lead = 0, last_e = SEQ_SINGLE, last_g = 0;
    // waves wholly past the end (short sums) skip the per-element work
    const bool wave_busy = __builtin_amdgcn_readfirstlane(len > 0 ? 1 : 0) != 0;
    if (wave_busy) {
        const double delta = (double)(c1 + 2) * 0x1p-23;
        const double mlo = 1.0 - delta, mhi = 1.0 + delta;
        // a chunk whose whole predicted range lies in one binade needs no
        // per-element binade checks
        const int ce_lo = dbl_exponent(P * mlo), ce_hi = dbl_exponent((P + loc) * mhi);
        const bool chunk_one = len > 0 && ce_lo == ce_hi && ce_lo > -89 && ce_lo < 99;
        if (chunk_one) {
            const float scale = pow2f(23 - ce_lo);
#pragma unroll
            for (int i = 0; i < MAXC; i++) {
                const float q = pr[i] * scale;  // p / u, exact
                const float fl = floorf(q);
                const float fr = q - fl;
                const bool ok = fr != 0.5f && fl < 16777216.0f;
                ec[i] = ok ? ce_lo : SEQ_SINGLE;
                g[i] = ok ? (int)fl + (fr > 0.5f ? 1 : 0) : 0;
            }
        } else {
#pragma unroll
            for (int i = 0; i < MAXC; i++) {
                const float p = pr[i];
                const double Pn = P + (double)p;
                const int elo = dbl_exponent(P * mlo), ehi = dbl_exponent(Pn * mhi);
                const int e = max(min(elo, 99), -89);
                const float q = p * pow2f(23 - e);  // p / u, exact
                const float fl = floorf(q);
                const float fr = q - fl;
                const bool ok = elo == ehi && elo == e && fr != 0.5f && fl < 16777216.0f;
                ec[i] = ok ? e : SEQ_SINGLE;
                g[i] = ok ? (int)fl + (fr > 0.5f ? 1 : 0) : 0;
                P = Pn;
            }
        }
        // run-local inclusive sums; the leading run of the chunk
        bool in_lead = ec[0] != SEQ_SINGLE;
#pragma unroll
        for (int i = 0; i < MAXC; i++) {
            if (i > 0) {
                const bool same = ec[i] != SEQ_SINGLE && ec[i] == ec[i - 1];
                g[i] = same ? g[i] + g[i - 1] : g[i];
                in_lead = in_lead && same;
            }
            lead += (in_lead && i < len) ? 1 : 0;
        }
#pragma unroll
        for (int i = 0; i < MAXC; i++)
            if (i == len - 1) {
                last_e = ec[i];
                last_g = g[i];
            }
    }
    SEQ_TS(5);
    if (act) {
        S.e_first[tid] = len > 0 ? ec[0] : SEQ_SINGLE;
        S.e_last[tid] = len > 0 ? last_e : SEQ_SINGLE;
    }
    __syncthreads();
    SEQ_TS(6);
    int cv = 0, cc = 0, total = 0, after_e = SEQ_SINGLE;
    bool cont = false;
    int v = 0, f = 1, c = 0;
    if (act) {
        const int before_e = tid > 0 ? S.e_last[tid - 1] : SEQ_SINGLE;
        after_e = (c1 < n && tid + 1 < T) ? S.e_first[tid + 1] : SEQ_SINGLE;
        cont = len > 0 && ec[0] != SEQ_SINGLE && ec[0] == before_e;
        // events ending in this chunk
        int n_end = 0;
#pragma unroll
        for (int i = 0; i < MAXC; i++) {
            const int next = i + 1 < len ? ec[i + 1 < MAXC ? i + 1 : i] : after_e;
            n_end += (i < len && (ec[i] == SEQ_SINGLE || next != ec[i])) ? 1 : 0;
        }
        // block scans: segmented run carry (v, f) and event offsets (c)
        v = last_g;
        f = (cont && lead == len) ? 0 : 1;
        c = n_end;
        if (len == 0) {
            v = 0;
            f = 1;
        }
        wave_scan_seg(v, f, c);
        SEQ_TS(7);
        if (lane == 63) {
            S.wv[wave] = v;
            S.wf[wave] = f;
            S.wc[wave] = c;
        }
    }
    __syncthreads();
    if (act) {
#pragma unroll
        for (int w = 0; w < NW; w++) {
            if (w < wave) {
                cv = S.wf[w] ? S.wv[w] : cv + S.wv[w];
                cc += S.wc[w];
            }
            total += S.wc[w];
        }
        const int pv = dpp_i<0x138, 0xf>(v), pf = dpp_i<0x138, 0xf>(f), pc = dpp_i<0x138, 0xf>(c);  // wave_shr:1
        cv = pf ? pv : cv + pv;  // run value flowing into this chunk
        cc += pc;                // events ending before this chunk
    } else {
#pragma unroll
        for (int w = 0; w < NW; w++) total += S.wc[w];
    }
    SEQ_TS(2);
    // 3. write the events at their slots
    const bool fits = total <= SEQ_MAX_EV;
    if (fits && act) {
        int slot = cc;
#pragma unroll
        for (int i = 0; i < MAXC; i++) {
            const int next = i + 1 < len ? ec[i + 1 < MAXC ? i + 1 : i] : after_e;
            if (i < len && (ec[i] == SEQ_SINGLE || next != ec[i])) {
                const int gt = g[i] + ((cont && i < lead) ? cv : 0);
                S.ev[slot] = make_int4(c0 + i, ec[i], gt, 0);
                slot++;
            }
        }
    }
    __syncthreads();
    SEQ_TS(3);
    // 4. walk on wave 0
    if (wave == 0) {
        float s = 0.0f;
        if (fits) {
            s = seq_walk<MAXC>(pp, C, total, S);
        } else {
            for (int k = 0; k < n; k++) s += pp[seq_idx(k, C)];
        }
        if (lane == 0) S.result = s;
    }
    __syncthreads();
    SEQ_TS(4);
    return S.result;
}

__device__ __forceinline__ float exact_seq_sum(const float *pp, int n, SeqScratch &S) {
    const int C = seq_chunk(n);
    if (seq_threads(n) == 256) return exact_seq_sum_t<4, 256>(pp, n, S);
    if (seq_threads(n) == 512) return exact_seq_sum_t<8, 512>(pp, n, S);
    if (C <= 4) return exact_seq_sum_t<4, SEQ_T>(pp, n, S);
    return exact_seq_sum_t<SEQ_MAX_N / SEQ_T, SEQ_T>(pp, n, S);
}

}  // namespace aotk
