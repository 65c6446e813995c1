// matvec.hip - batch-1 (and small-batch) quantized matrix-vector products on
// gfx950: matvec_<kind> / matvec3 / matvec2 / matmul of the reference
// (crates/aot-kernels/src/matvec.rs:300-583), bit-exact with its avx2+f16c
// kernels (simd_avx2.rs):
//   * K-quants: the per-super-block integer sums are exact (v_dot4 on
//     unpacked nibbles), then the f32 fold `sum += d*sumi - dmin*summ` runs
//     sequentially over super-blocks in the reference's order.
//   * Q8_0/Q4_0/Q5_0: the avx2 kernels keep 8 f32 lanes, lane l accumulating
//     fma(d*y.d, (f32) sum of products 4l..4l+3, acc_l) over blocks, then a
//     fixed horizontal sum; reproduced with 8 chains per row.
//   * F16/BF16/F32: 8 fma chains over 8-element groups, the same horizontal
//     sum, then the scalar tail.
// Weights are streamed once with 16-byte loads; the input vector is tiny and
// stays in L2/L1.
#include "actfn.hpp"
#include "device.hpp"
#include "internal.hpp"


#ifndef MV_TS
#define MV_TS(i)
#endif

namespace aotk {

constexpr int MAX_SEG = 3;

// Weight loads with the nontemporal hint (global_load ... nt): the weights are
// read once per token and streamed past the caches. Measured per kernel in the
// decode step: 426 -> 461 tok/s on Llama-3-8B, 990 -> 1085 on TinyLlama; the
// k_mv_kq rows of 10 and 40 super-blocks (Gemma-3's 2560 and 10240 columns)
// measured slower with it (4096x2560 Q5_K 4.3 -> 5.0 us) and keep plain loads.
// The hint pays only where each load instruction covers whole cache lines
// (the Q8_0 kernel's two 16-byte halves per block, with it: Qwen3 decode
// 234 -> 226 tok/s; hence its contiguous runs in k_mv_q8b).
typedef unsigned nt_u4 __attribute__((ext_vector_type(4)));
template <bool NT>
__device__ __forceinline__ uint4 ld_weights(const void *p) {
    if (!NT) return *(const uint4 *)p;
    const nt_u4 t = __builtin_nontemporal_load((const nt_u4 *)p);
    return make_uint4(t.x, t.y, t.z, t.w);
}
template <int NB>
constexpr bool kq_nt() { return NB > 0 && NB != 10 && NB != 40; }

struct MvArgs {
    const uint8_t *w[MAX_SEG];   // plane 0
    const uint8_t *w1[MAX_SEG];  // plane 1 (f16 scales) or null
    const uint8_t *w2[MAX_SEG];  // plane 2 (Q5_0 qh) or null
    float *y[MAX_SEG];
    const float *add[MAX_SEG];
    int rows[MAX_SEG];
    int nseg, total_rows;
    int nb;        // blocks per row
    size_t rb;     // bytes per row in plane 0 (row-major kinds)
    size_t cols;
    // activation (token t at offset t * cols / nb)
    const int8_t *xq;
    const float *xd;
    const int16_t *xbs;
    const float *xf;
    const int8_t *xt;  // Q8_K batches: the tiled copy of the quants (ActQ8K::qt)
    uint16_t *xh;  // Q8_0 family, batches: the quants as f16 (written by the batch's quantizer)
    // one token: when set, every block quantizes this f32 input itself
    // (K-quant rows to Q8_K, Q8_0 / Q4_0 / Q5_0 rows to Q8_0) instead of
    // reading xq / xd / xbs
    const float *xq_src;
};

// Ties v to this point of the program: loads before it stay before it and
// uses of v stay after it (a volatile asm with a memory clobber).
__device__ __forceinline__ void pin_after_loads(float4 &v) {
    float x = v.x, y = v.y, z = v.z, w = v.w;
    asm volatile("" : "+v"(x), "+v"(y), "+v"(z), "+v"(w) : : "memory");
    v = make_float4(x, y, z, w);
}

// Segment of a global row (constant indices only, so that the kernel
// arguments stay in scalar registers).
__device__ __forceinline__ int seg_of(const MvArgs &a, int row, int &local) {
    // selects, not branches: loads whose addresses depend on it stay in one
    // basic block, so the waits for them can stay exact
    const int r0 = a.rows[0], r1 = a.rows[1];
    const bool s1 = a.nseg > 1 && row >= r0;
    const bool s2 = a.nseg > 2 && row >= r0 + r1;
    local = row - (s2 ? r0 + r1 : (s1 ? r0 : 0));
    return s2 ? 2 : (s1 ? 1 : 0);
}
template <typename T>
__device__ __forceinline__ T seg_sel(int s, T v0, T v1, T v2) { return s == 0 ? v0 : (s == 1 ? v1 : v2); }

__device__ __forceinline__ void store_row(const MvArgs &a, int grow, int tok, float v) {
    int local;
    const int s = seg_of(a, grow, local);
    const size_t at = (size_t)tok * seg_sel(s, a.rows[0], a.rows[1], a.rows[2]) + local;
    const float *add = seg_sel(s, a.add[0], a.add[1], a.add[2]);
    const float r = add ? add[at] + v : v;
    seg_sel(s, a.y[0], a.y[1], a.y[2])[at] = r;
}

// --------------------------------------------------------------- K-quants
// Rows of more than 64 super-blocks (cols > 16384).
// Wave = R rows. Lane = 8*g + p: super-block slot g (8 per step), part p
// (32 of the block's 256 values). Each step's loads (activation slice, and per
// row the block header and 16 quant bytes, plus the high bits) are issued
// one step ahead of their use. Integer sums are reduced over the 8 lanes of
// a slot, then the per-super-block f32 terms are folded in order.
template <int KIND, int R>
struct KqLoads {
    uint4 ylo, yhi;
    float yd;
    int bslo, bshi;
    uint4 a[R];  // Q4_K/Q5_K: header;   Q6_K: ql
    uint4 q[R];  // Q4_K/Q5_K: quants;   Q6_K: qh
    uint4 h[R];  // Q5_K: qh;            Q6_K: scales 8n..8n+7 (x, y used)
    float d6[R]; // Q6_K: d
};

template <int KIND, int R>
__device__ __forceinline__ void kq_load(KqLoads<KIND, R> &L, const uint8_t *const wrow[R], const uint16_t *const drow[R],
                                        int nb, const int8_t *xq, const float *xd, const int16_t *xbs, int sbc, int p, int y_lo,
                                        int y_hi, int bs_lo, int bs_hi) {
    L.ylo = *(const uint4 *)(xq + (size_t)sbc * 256 + y_lo);
    L.yhi = *(const uint4 *)(xq + (size_t)sbc * 256 + y_hi);
    L.yd = xd[sbc];
    L.bslo = xbs[(size_t)sbc * 16 + bs_lo];
    L.bshi = xbs[(size_t)sbc * 16 + bs_hi];
#pragma unroll
    for (int r = 0; r < R; r++) {
        const uint8_t *b = wrow[r] + (size_t)sbc * 16;  // chunk-major rows
        const size_t cs = (size_t)nb * 16;                // stride of one chunk index
        if (KIND == AOTK_Q4_K || KIND == AOTK_Q5_K) {
            constexpr int QC = KIND == AOTK_Q4_K ? 1 : 3;
            L.a[r] = *(const uint4 *)b;
            L.q[r] = *(const uint4 *)(b + (QC + p) * cs);
            if (KIND == AOTK_Q5_K) L.h[r] = *(const uint4 *)(b + (1 + (p & 1)) * cs);
        } else {
            const int n = p >> 2, half = (p >> 1) & 1, which = p & 1;
            L.a[r] = *(const uint4 *)(b + (4 * n + 2 * which + half) * cs);
            L.q[r] = *(const uint4 *)(b + (8 + 2 * n + half) * cs);
            uint2 sc = *(const uint2 *)(b + 12 * cs + 8 * n);
            L.h[r] = make_uint4(sc.x, sc.y, 0, 0);
            L.d6[r] = f16_to_f32(drow[r][sbc]);
        }
    }
}

template <int KIND, int R>
__global__ __launch_bounds__(256) void k_mv_kquant(MvArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int tok = blockIdx.y;
    const int grow0 = (blockIdx.x * 4 + wave) * R;
    if (grow0 >= a.total_rows) return;
    const int g = lane >> 3, p = lane & 7;
    const int nb = a.nb;
    const int8_t *xq = a.xq + (size_t)tok * a.cols;
    const float *xd = a.xd + (size_t)tok * nb;
    const int16_t *xbs = a.xbs + (size_t)tok * nb * 16;

    const uint8_t *wrow[R];
    const uint16_t *drow[R];
    bool rvalid[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        int grow = grow0 + r;
        rvalid[r] = grow < a.total_rows;
        int local;
        int s = seg_of(a, rvalid[r] ? grow : grow0, local);
        if (KIND == AOTK_Q6_K) {
            wrow[r] = seg_sel(s, a.w[0], a.w[1], a.w[2]) + (size_t)local * nb * 208;
            drow[r] = (const uint16_t *)seg_sel(s, a.w1[0], a.w1[1], a.w1[2]) + (size_t)local * nb;
        } else {
            wrow[r] = seg_sel(s, a.w[0], a.w[1], a.w[2]) + (size_t)local * a.rb;
            drow[r] = nullptr;
        }
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;

    // lane-constant geometry
    int y_lo, y_hi, bs_lo, bs_hi;
    if (KIND == AOTK_Q6_K) {
        const int n = p >> 2, half = (p >> 1) & 1, which = p & 1;
        y_lo = 128 * n + 32 * which + 16 * half;
        y_hi = y_lo + 64;
        bs_lo = y_lo / 16;
        bs_hi = y_hi / 16;
    } else {
        const int j = p >> 1, h = p & 1;
        y_lo = 64 * j + 16 * h;
        y_hi = y_lo + 32;
        bs_lo = 4 * j + h;
        bs_hi = bs_lo + 2;
    }

    KqLoads<KIND, R> cur;
    kq_load<KIND, R>(cur, wrow, drow, nb, xq, xd, xbs, g < nb ? g : nb - 1, p, y_lo, y_hi, bs_lo, bs_hi);
    for (int sb0 = 0; sb0 < nb; sb0 += 8) {
        KqLoads<KIND, R> nxt;
        const bool more = sb0 + 8 < nb;
        if (more) {
            const int sbn = sb0 + 8 + g;
            kq_load<KIND, R>(nxt, wrow, drow, nb, xq, xd, xbs, sbn < nb ? sbn : nb - 1, p, y_lo, y_hi, bs_lo, bs_hi);
        }
        const uint32_t ylw[4] = {cur.ylo.x, cur.ylo.y, cur.ylo.z, cur.ylo.w};
        const uint32_t yhw[4] = {cur.yhi.x, cur.yhi.y, cur.yhi.z, cur.yhi.w};
        const int nstep = nb - sb0 < 8 ? nb - sb0 : 8;
#pragma unroll
        for (int r = 0; r < R; r++) {
            int sumi = 0, summ = 0;
            float dd, dm = 0.0f;
            if (KIND == AOTK_Q4_K || KIND == AOTK_Q5_K) {
                const uint4 hdr = cur.a[r];
                const int j = p >> 1;
                int sc_lo, m_lo, sc_hi, m_hi;
                scale_min_k4(2 * j, hdr.y, hdr.z, hdr.w, sc_lo, m_lo);
                scale_min_k4(2 * j + 1, hdr.y, hdr.z, hdr.w, sc_hi, m_hi);
                const uint32_t qw[4] = {cur.q[r].x, cur.q[r].y, cur.q[r].z, cur.q[r].w};
                const uint32_t hw[4] = {cur.h[r].x, cur.h[r].y, cur.h[r].z, cur.h[r].w};
                int slo = 0, shi = 0;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    uint32_t lo = qw[k] & 0x0F0F0F0Fu;
                    uint32_t hi = (qw[k] >> 4) & 0x0F0F0F0Fu;
                    if (KIND == AOTK_Q5_K) {
                        lo |= ((hw[k] >> (2 * j)) & 0x01010101u) << 4;
                        hi |= ((hw[k] >> (2 * j + 1)) & 0x01010101u) << 4;
                    }
                    slo = dot4(lo, ylw[k], slo);
                    shi = dot4(hi, yhw[k], shi);
                }
                sumi = sc_lo * slo + sc_hi * shi;
                summ = m_lo * cur.bslo + m_hi * cur.bshi;
                dd = f16_to_f32(hdr.x & 0xFFFFu) * cur.yd;
                dm = f16_to_f32(hdr.x >> 16) * cur.yd;
            } else {  // Q6_K
                const int half = (p >> 1) & 1, which = p & 1;
                const int is_lo = half + 2 * which, is_hi = is_lo + 4;
                const uint32_t scw = is_lo < 4 ? cur.h[r].x : cur.h[r].y;
                const uint32_t scw2 = cur.h[r].y;
                const int sc_lo = (int)(int8_t)((scw >> (8 * (is_lo & 3))) & 0xFFu);
                const int sc_hi = (int)(int8_t)((scw2 >> (8 * (is_hi & 3))) & 0xFFu);
                const int sh_lo = 2 * which, sh_hi = 4 + 2 * which;
                const uint32_t lw[4] = {cur.a[r].x, cur.a[r].y, cur.a[r].z, cur.a[r].w};
                const uint32_t hw[4] = {cur.q[r].x, cur.q[r].y, cur.q[r].z, cur.q[r].w};
                int slo = 0, shi = 0;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    uint32_t lo = (lw[k] & 0x0F0F0F0Fu) | (((hw[k] >> sh_lo) & 0x03030303u) << 4);
                    uint32_t hi = ((lw[k] >> 4) & 0x0F0F0F0Fu) | (((hw[k] >> sh_hi) & 0x03030303u) << 4);
                    slo = dot4(lo, ylw[k], slo);
                    shi = dot4(hi, yhw[k], shi);
                }
                // unsigned 6-bit values: subtract 32 * sum(y) per 16-group.
                sumi = sc_lo * (slo - 32 * cur.bslo) + sc_hi * (shi - 32 * cur.bshi);
                dd = cur.d6[r] * cur.yd;
            }
            // exact integer reduction over the 8 parts of the super-block
            sumi += shfl_xor(sumi, 1);
            sumi += shfl_xor(sumi, 2);
            sumi += shfl_xor(sumi, 4);
            float term;
            if (KIND == AOTK_Q6_K) {
                term = dd * (float)sumi;
            } else {
                summ += shfl_xor(summ, 1);
                summ += shfl_xor(summ, 2);
                summ += shfl_xor(summ, 4);
                term = dd * (float)sumi - dm * (float)summ;
            }
            // sequential fold over the super-blocks of this step
            float s_acc = acc[r];
            for (int gg = 0; gg < nstep; gg++) s_acc = s_acc + readlane_f(term, gg * 8);
            acc[r] = s_acc;
        }
        if (more) cur = nxt;
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; r++)
            if (rvalid[r]) store_row(a, grow0 + r, tok, acc[r]);
    }
}

// Rows of at most 64 super-blocks: lane = (row slot rs, super-block s),
// RL row slots of nb lanes per wave. A lane holds the activation of its
// super-block in registers for all its rows, loads its super-block's
// chunks (each chunk index is one contiguous run over the row, see the
// chunk-major layout), and computes the exact integer sums and the f32 term
// d*sumi - dmin*summ alone. The row's terms are then folded in super-block
// order by one lane through LDS. A wave does G row groups, the next group's
// weights in flight while the current one is computed.
template <int KIND>
struct KqGeom {
    static constexpr int CH = KIND == AOTK_Q4_K ? 9 : (KIND == AOTK_Q5_K ? 11 : 13);  // 16-byte chunks
    static constexpr int RB = KIND == AOTK_Q4_K ? 144 : (KIND == AOTK_Q5_K ? 176 : 208);  // plane-0 bytes
};


// Activation record of one super-block in LDS: qs (256 B), bsums (32 B), d,
// padded to 304 B so that the lanes of a 16-lane group reading their own
// super-block's record with 16-byte loads hit disjoint banks.
constexpr int KQ_REC = 304;

// Rows of <= 32 super-blocks split each super-block over two lanes (SPL = 2):
// lane h of the pair takes the first or the second half of the 256 values
// (Q4_K/Q5_K sub-blocks 4h..4h+3, Q6_K 16-value groups 8h..8h+7), the pair
// adds its integer sums (exact, so the split changes nothing) and both form
// the f32 term. The chunks a lane holds, in the order kq_sums reads them:
//   Q4_K: header, then the 4 qs chunks of its half;
//   Q5_K: header, the 2 qh chunks, the 4 qs chunks of its half;
//   Q6_K: the 4 ql chunks and 2 qh chunks of its half, the scales.
template <int KIND, int SPL>
__device__ __forceinline__ constexpr int kq_chl() {
    return SPL == 1 ? KqGeom<KIND>::CH : (KIND == AOTK_Q4_K ? 5 : 7);
}
template <int KIND, int SPL>
__device__ __forceinline__ int kq_chunk(int k, int h) {
    if (SPL == 1) return k;
    if (KIND == AOTK_Q4_K) return k == 0 ? 0 : 1 + 4 * h + (k - 1);
    if (KIND == AOTK_Q5_K) return k < 3 ? k : 3 + 4 * h + (k - 3);
    return k < 4 ? 4 * h + k : (k < 6 ? 8 + 2 * h + (k - 4) : 12);
}

// The exact integer sums of one lane's share of a super-block (sumi: the
// scaled dot products; summ: the mins against the bsums) and, after the
// pair's exchange, the f32 term d*sumi - dmin*summ of quant.rs/matvec.rs.
template <int KIND, int SPL>
__device__ __forceinline__ float kq_term(const uint4 (&c)[kq_chl<KIND, SPL>()], float d6, const uint8_t *rec, int h) {
    const float yd = *(const float *)(rec + 288);
    const uint8_t *rh = rec + 128 * h;  // this lane's half of the activation
    constexpr int NBW = 8 / SPL;         // bsum words of the lane's share
    uint32_t bw[NBW];
#pragma unroll
    for (int q = 0; q < NBW / 4; q++) {
        const uint4 b = *(const uint4 *)(rec + 256 + 16 * (h * (NBW / 4) + q));
        bw[4 * q] = b.x;
        bw[4 * q + 1] = b.y;
        bw[4 * q + 2] = b.z;
        bw[4 * q + 3] = b.w;
    }
    auto bs = [&](int g) { return (int)(int16_t)((bw[g >> 1] >> (16 * (g & 1))) & 0xFFFFu); };  // local group
    int sumi = 0;
    if (KIND == AOTK_Q4_K || KIND == AOTK_Q5_K) {
        constexpr int QC = KIND == AOTK_Q4_K ? 1 : 3;
        constexpr int NJ = 4 / SPL;  // 64-value sub-block pairs of the lane
        const uint4 hdr = c[0];
        int summ = 0;
        uint32_t hq[8];
        if (KIND == AOTK_Q5_K) {
            const int sh = 2 * NJ * h;  // the qh bits of the lane's first pair
            hq[0] = c[1].x >> sh; hq[1] = c[1].y >> sh; hq[2] = c[1].z >> sh; hq[3] = c[1].w >> sh;
            hq[4] = c[2].x >> sh; hq[5] = c[2].y >> sh; hq[6] = c[2].z >> sh; hq[7] = c[2].w >> sh;
        }
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const uint4 q0 = c[QC + 2 * j], q1 = c[QC + 2 * j + 1];
            const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
            const uint4 l0 = *(const uint4 *)(rh + 64 * j), l1 = *(const uint4 *)(rh + 64 * j + 16);
            const uint4 h0 = *(const uint4 *)(rh + 64 * j + 32), h1 = *(const uint4 *)(rh + 64 * j + 48);
            const uint32_t yl[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
            const uint32_t yh[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
            int slo = 0, shi = 0;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                uint32_t lo = qw[k] & 0x0F0F0F0Fu;
                uint32_t hi = (qw[k] >> 4) & 0x0F0F0F0Fu;
                if (KIND == AOTK_Q5_K) {
                    lo |= ((hq[k] >> (2 * j)) & 0x01010101u) << 4;
                    hi |= ((hq[k] >> (2 * j + 1)) & 0x01010101u) << 4;
                }
                slo = dot4(lo, yl[k], slo);
                shi = dot4(hi, yh[k], shi);
            }
            int sc0, m0, sc1, m1;
            if (SPL == 1) {
                scale_min_k4(2 * j, hdr.y, hdr.z, hdr.w, sc0, m0);
                scale_min_k4(2 * j + 1, hdr.y, hdr.z, hdr.w, sc1, m1);
            } else {  // sub-blocks 2j, 2j + 1 of the lane's half: 4h + 2j, 4h + 2j + 1
                int a0, b0, a1, b1, c0, e0, c1, e1;
                scale_min_k4(2 * j, hdr.y, hdr.z, hdr.w, a0, b0);
                scale_min_k4(2 * j + 1, hdr.y, hdr.z, hdr.w, a1, b1);
                scale_min_k4(4 + 2 * j, hdr.y, hdr.z, hdr.w, c0, e0);
                scale_min_k4(4 + 2 * j + 1, hdr.y, hdr.z, hdr.w, c1, e1);
                sc0 = h ? c0 : a0;
                m0 = h ? e0 : b0;
                sc1 = h ? c1 : a1;
                m1 = h ? e1 : b1;
            }
            // 24-bit multiplies (full rate): every factor fits in 24 bits
            sumi += __mul24(sc0, slo) + __mul24(sc1, shi);
            summ += __mul24(m0, bs(4 * j) + bs(4 * j + 1)) + __mul24(m1, bs(4 * j + 2) + bs(4 * j + 3));
            asm volatile("" ::: "memory");  // keep the activation reads local
        }
        if (SPL == 2) {
            sumi += dppx_i<DPP_XOR1>(sumi);
            summ += dppx_i<DPP_XOR1>(summ);
        }
        const float dd = f16_to_f32(hdr.x & 0xFFFFu) * yd;
        const float dm = f16_to_f32(hdr.x >> 16) * yd;
        return dd * (float)sumi - dm * (float)summ;
    } else {
        constexpr int NG = 16 / SPL;  // 16-value groups of the lane
        const uint4 scv = c[kq_chl<KIND, SPL>() - 1];
        uint32_t scw[NG / 4];
        if (SPL == 1) {
            scw[0] = scv.x; scw[1] = scv.y; scw[NG / 4 - 2] = scv.z; scw[NG / 4 - 1] = scv.w;
        } else {
            scw[0] = h ? scv.z : scv.x;
            scw[1] = h ? scv.w : scv.y;
        }
#pragma unroll
        for (int g = 0; g < NG; g++) {
            const int n = g >> 3, quarter = (g & 7) >> 1, half = g & 1;
            const uint4 l4 = SPL == 1 ? c[4 * n + 2 * (quarter & 1) + half] : c[2 * (quarter & 1) + half];
            const uint4 h4 = SPL == 1 ? c[8 + 2 * n + half] : c[4 + half];
            const uint4 y4 = *(const uint4 *)(rh + 16 * g);
            const uint32_t lw[4] = {l4.x, l4.y, l4.z, l4.w};
            const uint32_t hw[4] = {h4.x, h4.y, h4.z, h4.w};
            const uint32_t yw[4] = {y4.x, y4.y, y4.z, y4.w};
            int sg = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint32_t nib = quarter >= 2 ? (lw[k] >> 4) & 0x0F0F0F0Fu : lw[k] & 0x0F0F0F0Fu;
                const uint32_t v = nib | (((hw[k] >> (2 * quarter)) & 0x03030303u) << 4);
                sg = dot4(v, yw[k], sg);
            }
            const int sc = (int)(int8_t)((scw[g >> 2] >> (8 * (g & 3))) & 0xFFu);
            sumi += __mul24(sc, sg - 32 * bs(g));  // |sg - 32 bs| < 2^18
            if ((g & 3) == 3) asm volatile("" ::: "memory");  // keep the activation reads local
        }
        if (SPL == 2) sumi += dppx_i<DPP_XOR1>(sumi);
        const float dd = d6 * yd;
        return dd * (float)sumi;
    }
}

// Lanes per super-block: two for the row widths with their own
// instantiation up to 32 super-blocks, else one.
__host__ __device__ constexpr int kq_spl(int nb) { return nb > 0 && nb <= 32 ? 2 : 1; }

// PF = 0: one row group per wave (G == 1), no second register set;
// PF = 1: G groups per wave with the next group's loads in flight while the
// current one computes (launched with G == 1 for Q6_K rows of one lane per
// super-block and for the f32-input variant, whose register budget of two
// waves per SIMD measured faster there).
// NB > 0: the super-blocks per row as a compile-time constant (immediate
// chunk offsets, constant row-slot division, an unmasked fold); NB == 0 reads
// it from the arguments.
template <int KIND, int PF, int NB, bool QSRC = false>
__device__ __forceinline__ void mv_kq_body(const MvArgs &a, int RL, int G, int bx, uint8_t *sY, float (*sT)[256 + 16]) {
    using Geo = KqGeom<KIND>;
    constexpr int SPL = kq_spl(NB);
    constexpr int CH = kq_chl<KIND, SPL>();
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tok = blockIdx.y;
    const int nb = NB > 0 ? NB : a.nb;
    if (NB > 0) RL = 64 / (SPL * NB);
    const int h = SPL == 2 ? lane & 1 : 0;  // half of the super-block
    const int li = SPL == 2 ? lane >> 1 : lane;
    const int rs = li / nb, s = li - rs * nb;
    const bool lane_on = rs < RL;
    const int sa = lane_on ? s : 0;
    const size_t cs = (size_t)nb * 16;
    const size_t rowb = (size_t)nb * Geo::RB;
    const int group0 = (bx * 4 + wave) * G;
    const int ts = (nb + 3) & ~3;  // row stride of the fold buffer (RL * ts <= 256)

    uint4 cur[CH], nxt[PF ? CH : 1];
    float dcur = 0.0f, dnxt = 0.0f;
    auto load = [&](uint4 *c, float &d6, int gi) {
        // rows past the end load row 0 (valid memory); their results are
        // never folded
        const int row = (group0 + gi) * RL + rs;
        const bool on = lane_on && row < a.total_rows;
        int local;
        const int sg = seg_of(a, on ? row : 0, local);
        const uint8_t *wp = seg_sel(sg, a.w[0], a.w[1], a.w[2]) + (size_t)local * rowb + (size_t)sa * 16;
#pragma unroll
        for (int k = 0; k < CH; k++) c[k] = ld_weights<kq_nt<NB>()>(wp + kq_chunk<KIND, SPL>(k, h) * cs);
        if (KIND == AOTK_Q6_K)
            d6 = f16_to_f32(((const uint16_t *)seg_sel(sg, a.w1[0], a.w1[1], a.w1[2]))[(size_t)local * nb + sa]);
    };
    MV_TS(0);
    // This token's Q8_K activation is loaded first (<= 64 super-blocks: four
    // quads of qs, one of bsums and one scale per thread; indices past the
    // end repeat the last element), then the weights of the first group:
    // waiting for the activation then leaves the weights in flight.
    constexpr bool stage = !QSRC;  // QSRC: the input arrives in f32 (a.xq_src) and is quantized here
    const int nq = nb * 16;
    uint4 xv[4], bv;
    float dv;
    float4 xf[4];  // the f32 input of the wave's first four super-blocks, when it quantizes
    if constexpr (stage) {
        const uint4 *xq = (const uint4 *)(a.xq + (size_t)tok * a.cols);
        const uint4 *xb = (const uint4 *)(a.xbs + (size_t)tok * nb * 16);
#pragma unroll
        for (int k = 0; k < 4; k++) xv[k] = xq[min(tid + 256 * k, nq - 1)];
        bv = xb[min(tid, 2 * nb - 1)];
        dv = a.xd[(size_t)tok * nb + min(tid, nb - 1)];
    } else {
#pragma unroll
        for (int k = 0; k < 4; k++) xf[k] = ((const float4 *)(a.xq_src + (size_t)min(wave + 4 * k, nb - 1) * 256))[lane];
    }
    load(cur, dcur, 0);
    // the f32 input's loads stay ahead of the weights' and its quantization
    // after them (no code motion across this point): the quantizer then
    // waits for the input only, with the weights in flight
    if constexpr (!stage)
#pragma unroll
        for (int k = 0; k < 4; k++) pin_after_loads(xf[k]);
    if constexpr (stage) {
        // unconditional stores: past the end they repeat the last element
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int i = min(tid + 256 * k, nq - 1);
            *(uint4 *)(sY + (i >> 4) * KQ_REC + (i & 15) * 16) = xv[k];
        }
        const int ib = min(tid, 2 * nb - 1);
        *(uint4 *)(sY + (ib >> 1) * KQ_REC + 256 + (ib & 1) * 16) = bv;
        *(float *)(sY + min(tid, nb - 1) * KQ_REC + 288) = dv;
    } else {
        // quantize the f32 input here, wave w taking super-blocks w, w + 4,
        // ... (the device quantizer of k_quant_f32, quant.rs:248-283)
        // The first four super-blocks of the wave come from the loads issued
        // before the weights' (xf); later ones are loaded here. (A select
        // between xf and a load makes the load unconditional, after the
        // weights', and the wait for it then waits for the weights too.)
        for (int b0 = wave; b0 < nb; b0 += 16) {
            float4 v4[4];  // four super-blocks' loads in flight together
            if (b0 == wave) {
#pragma unroll
                for (int k = 0; k < 4; k++) v4[k] = xf[k];
            } else {
#pragma unroll
                for (int k = 0; k < 4; k++) v4[k] = ((const float4 *)(a.xq_src + (size_t)min(b0 + 4 * k, nb - 1) * 256))[lane];
            }
            Q8KLane rq[4];  // independent: their reductions interleave
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float v[4] = {v4[k].x, v4[k].y, v4[k].z, v4[k].w};
                rq[k] = q8k_lane(v, lane);
            }
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int b = b0 + 4 * k;
                if (b >= nb) break;
                const Q8KLane &r = rq[k];
                uint8_t *recb = sY + b * KQ_REC;
                ((uint32_t *)recb)[lane] = r.packed;
                if ((lane & 3) == 0) ((int16_t *)(recb + 256))[lane >> 2] = (int16_t)r.quad_sum;
                if (lane == 0) *(float *)(recb + 288) = r.d;
            }
        }
    }
    __syncthreads();
    MV_TS(1);
    const uint8_t *rec = sY + sa * KQ_REC;
    const int ng = PF ? G : 1;
    // one row group: the term, the fold in super-block order (terms read 16
    // at a time ahead of the dependent adds), the store
    auto group = [&](const uint4 *c, float d6, int gi) {
        const int gr0 = (group0 + gi) * RL;
        const float term = kq_term<KIND, SPL>(*(const uint4(*)[CH])c, d6, rec, h);
        MV_TS(2 + 2 * gi);
        if (lane_on && h == 0) sT[wave][rs * ts + s] = term;
        wave_lds_sync();
        if (lane < RL && gr0 + lane < a.total_rows) {
            const float4 *tp = (const float4 *)&sT[wave][lane * ts];
            float acc = 0.0f;
            for (int k0 = 0; k0 < nb; k0 += 16) {
                float t[16];
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const float4 v = tp[k0 / 4 + q];
                    t[4 * q] = v.x;
                    t[4 * q + 1] = v.y;
                    t[4 * q + 2] = v.z;
                    t[4 * q + 3] = v.w;
                }
                const int n = nb - k0 < 16 ? nb - k0 : 16;
#pragma unroll
                for (int q = 0; q < 16; q++)
                    if (q < n) acc = acc + t[q];
            }
            store_row(a, gr0 + lane, tok, acc);
        }
        wave_lds_sync();
        MV_TS(3 + 2 * gi);
    };
    // groups alternate between the two register buffers (no copies)
    for (int gi = 0; gi < ng; gi += 2) {
        if ((group0 + gi) * RL >= a.total_rows) break;
        if (PF && gi + 1 < ng) load(nxt, dnxt, gi + 1);
        group(cur, dcur, gi);
        if (!PF || gi + 1 >= ng || (group0 + gi + 1) * RL >= a.total_rows) break;
        if (gi + 2 < ng) load(cur, dcur, gi + 2);
        group(nxt, dnxt, gi + 1);
    }
}

// LDS of one K-quant block: the activation records (one per super-block of
// the row; sized to NB when it is known, so that short rows leave room for
// more resident blocks) and the fold buffer.
template <int NB>
struct KqShared {
    __align__(16) uint8_t y[(NB > 0 ? NB : 64) * KQ_REC];
    __align__(16) float t[4][256 + 16];  // [wave][row slot * ts + super-block] (+ read slack)
};

template <int KIND, int PF, int NB, bool QSRC = false>
__global__ __launch_bounds__(256, PF ? 2 : 4) void k_mv_kq(MvArgs a, int RL, int G) {
    __shared__ KqShared<NB> sh;
    mv_kq_body<KIND, PF, NB, QSRC>(a, RL, G, blockIdx.x, sh.y, sh.t);
}

// Two K-quant matrices of different kinds sharing the input in one launch
// (q/k in one kind and v in another): blocks [0, nblk_a) run `a`, the rest
// run `b`.
// PF as for mv_kq_body (launched with PF == 0).
template <int KA, int KB, int NB, int PF>
__global__ __launch_bounds__(256, PF ? 2 : 4) void k_mv_kq2(MvArgs a, int RLa, int Ga, MvArgs b, int RLb, int Gb, int nblk_a) {
    __shared__ KqShared<NB> sh;
    if ((int)blockIdx.x < nblk_a) mv_kq_body<KA, PF, NB>(a, RLa, Ga, blockIdx.x, sh.y, sh.t);
    else mv_kq_body<KB, PF, NB>(b, RLb, Gb, blockIdx.x - nblk_a, sh.y, sh.t);
}

// Rows of 33..64 super-blocks on two waves each: wave 2r + w of the block
// takes super-blocks 32w .. 32w + 31 of row r, each split over a lane pair
// as for short rows (the same SPL = 2 term); the terms meet in LDS and one
// lane folds the row in super-block order. Half the per-lane work of one
// lane per whole super-block, on twice the waves (Q6_K 4096x14336: 11.9
// against 13.5 us).
template <int KIND, int NB>
__global__ __launch_bounds__(256) void k_mv_kqw(MvArgs a) {
    static_assert(NB > 32 && NB <= 64, "rows of 33..64 super-blocks");
    __shared__ __align__(16) uint8_t sY[NB * KQ_REC];
    __shared__ __align__(16) float sT[2][64];
    using Geo = KqGeom<KIND>;
    constexpr int CH = kq_chl<KIND, 2>();
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tok = blockIdx.y;
    const int h = lane & 1;
    const int s = 32 * (wave & 1) + (lane >> 1);
    const bool lane_on = s < NB;
    const int sa = lane_on ? s : 0;
    const int rslot = wave >> 1;
    const int row = blockIdx.x * 2 + rslot;
    const bool row_on = row < a.total_rows;
    constexpr size_t cs = (size_t)NB * 16;
    constexpr size_t rowb = (size_t)NB * Geo::RB;
    // the activation first (as mv_kq_body), then the weights
    constexpr int nq = NB * 16;
    const uint4 *xq = (const uint4 *)(a.xq + (size_t)tok * a.cols);
    const uint4 *xb = (const uint4 *)(a.xbs + (size_t)tok * NB * 16);
    uint4 xv[4];
#pragma unroll
    for (int k = 0; k < 4; k++) xv[k] = xq[min(tid + 256 * k, nq - 1)];
    const uint4 bv = xb[min(tid, 2 * NB - 1)];
    const float dv = a.xd[(size_t)tok * NB + min(tid, NB - 1)];
    // rows past the end load row 0 (valid memory); they are never stored
    int local;
    const int sg = seg_of(a, row_on ? row : 0, local);
    const uint8_t *wp = seg_sel(sg, a.w[0], a.w[1], a.w[2]) + (size_t)local * rowb + (size_t)sa * 16;
    uint4 c[CH];
#pragma unroll
    for (int k = 0; k < CH; k++) c[k] = ld_weights<true>(wp + kq_chunk<KIND, 2>(k, h) * cs);
    float d6 = 0.0f;
    if (KIND == AOTK_Q6_K) d6 = f16_to_f32(((const uint16_t *)seg_sel(sg, a.w1[0], a.w1[1], a.w1[2]))[(size_t)local * NB + sa]);
    // unconditional stores: past the end they repeat the last element
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int i = min(tid + 256 * k, nq - 1);
        *(uint4 *)(sY + (i >> 4) * KQ_REC + (i & 15) * 16) = xv[k];
    }
    const int ib = min(tid, 2 * NB - 1);
    *(uint4 *)(sY + (ib >> 1) * KQ_REC + 256 + (ib & 1) * 16) = bv;
    *(float *)(sY + min(tid, NB - 1) * KQ_REC + 288) = dv;
    __syncthreads();
    const float term = kq_term<KIND, 2>(c, d6, sY + sa * KQ_REC, h);
    if (lane_on && h == 0) sT[rslot][s] = term;
    __syncthreads();
    if ((wave & 1) == 0 && lane == 0 && row_on) {
        const float4 *tp = (const float4 *)sT[rslot];
        float acc = 0.0f;
#pragma unroll
        for (int q = 0; q < (NB + 3) / 4; q++) {
            const float4 v = tp[q];
            acc = acc + v.x;
            if (4 * q + 1 < NB) acc = acc + v.y;
            if (4 * q + 2 < NB) acc = acc + v.z;
            if (4 * q + 3 < NB) acc = acc + v.w;
        }
        store_row(a, row, tok, acc);
    }
}

// The row lengths of the configs (cols / 256) get their own instantiations.
#define AOTK_NB_SWITCH(nb, F) \
    switch (nb) {             \
    case 8: F(8); break;      \
    case 10: F(10); break;    \
    case 16: F(16); break;    \
    case 22: F(22); break;    \
    case 40: F(40); break;    \
    case 48: F(48); break;    \
    case 56: F(56); break;    \
    default: F(0); break;     \
    }

// ------------------------------------------------- K-quant matmul (MFMA)
// Prompt batches (m tokens, 2 <= m <= 64): block = 16 weight rows x 64
// tokens, wave w taking the 16-token tile w. Per super-block, v_mfma_i32_16x16x32_i8 computes exact
// integer dot products of 32 values: A = activations (16 tokens x 32 k),
// B = the quants of the wave's 16 rows (32 k x 16 rows), so lane l owns
// weight row l % 16 and tokens 4*(l/16) + i of each 16-token tile. Per
// sub-block the integer sums are scaled by the lane's row scale (exact
// integer arithmetic) and, for Q4_K/Q5_K, summ = sum m_j * y is accumulated by
// a second MFMA with the mins broadcast. The f32 fold per super-block is the
// same expression, in the same order, as the matvec (bit-identical to m
// matvecs, matvec.rs:479-583). Activations are staged per super-block in LDS
// (double-buffered), the next super-block's quants are loaded ahead.
typedef int mm_v4i __attribute__((ext_vector_type(4)));
constexpr int MM_TOK = 64;        // tokens per block (4 tiles of 16)
constexpr int MM_MIN_TOKENS = 2;  // smaller batches use the matvec kernels
constexpr int MM_YS = 256 + 8;    // LDS bytes per token row of one super-block (padded)

template <int KIND>
struct MmW {
    uint4 hdr;      // Q4_K/Q5_K: d, dmin, scales; Q6_K: the 16 scales
    uint2 q[4];     // Q4_K/Q5_K: qs bytes for sub-block pairs; Q6_K: ql bytes for j = 0..3 ...
    uint2 q2[4];    // Q5_K: qh bytes (pairs); Q6_K: ql bytes for j = 4..7
    uint2 h6[8];    // Q6_K: qh bytes per j
    float d6;
};

// Load the lane's share of super-block sb of row `row`: for each 32-value
// step j, the 8 values k = 32j + 8q .. +8 (q = lane / 16).
template <int KIND>
__device__ __forceinline__ void mm_load(MmW<KIND> &w, const uint8_t *rowp, const uint16_t *drow, int sb, int nb, int q) {
    const size_t cs = (size_t)nb * 16;
    const uint8_t *b = rowp + (size_t)sb * 16;
    if (KIND == AOTK_Q4_K || KIND == AOTK_Q5_K) {
        constexpr int QC = KIND == AOTK_Q4_K ? 1 : 3;
        w.hdr = *(const uint4 *)b;
        // pair p (sub-blocks 2p, 2p+1): qs bytes 32p + 8q .. +8 -> chunk QC + 2p + q/2, offset 8*(q%2)
#pragma unroll
        for (int p = 0; p < 4; p++) w.q[p] = *(const uint2 *)(b + (QC + 2 * p + (q >> 1)) * cs + 8 * (q & 1));
        if (KIND == AOTK_Q5_K)  // qh bytes 8q .. +8 -> chunk 1 + q/2
#pragma unroll
            for (int p = 0; p < 4; p++) w.q2[p] = *(const uint2 *)(b + (1 + (q >> 1)) * cs + 8 * (q & 1));
    } else {
        w.hdr = *(const uint4 *)(b + 12 * cs);
        w.d6 = f16_to_f32(drow[sb]);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            // k0 = 32j + 8q: half n = j/4, quarter = j%4, l = 8q
            const int n = j >> 2, quarter = j & 3;
            const int qlo = 64 * n + 8 * q + 32 * (quarter & 1);  // ql byte offset
            const int qho = 128 + 32 * n + 8 * q;                  // qh byte offset
            const uint2 lo = *(const uint2 *)(b + (qlo >> 4) * cs + (qlo & 15));
            if (j < 4) w.q[j] = lo;
            else w.q2[j - 4] = lo;
            w.h6[j] = *(const uint2 *)(b + (qho >> 4) * cs + (qho & 15));
        }
    }
}

// The B side of one super-block of the 16 rows of a wave, unpacked once and
// shared by every token tile: the lane's 8 quant values of each 32-value
// step j (k = 32j + 8q .. +8, as signed int8; Q6_K with the -32 offset
// applied), the row's scales and, for Q4_K/Q5_K, the mins broadcast to the
// 8 values of a step.
template <int KIND>
struct MmB {
    long bq[8];
    int sc[16];
    int mn[8];
    float dd, dm;
};

template <int KIND>
__device__ __forceinline__ void mm_prep(const MmW<KIND> &cur, MmB<KIND> &b) {
    if (KIND == AOTK_Q6_K) {
        const uint32_t scw[4] = {cur.hdr.x, cur.hdr.y, cur.hdr.z, cur.hdr.w};
#pragma unroll
        for (int g = 0; g < 16; g++) b.sc[g] = (int)(int8_t)((scw[g >> 2] >> (8 * (g & 3))) & 0xFFu);
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) scale_min_k4(j, cur.hdr.y, cur.hdr.z, cur.hdr.w, b.sc[j], b.mn[j]);
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
        uint32_t w0, w1;
        if (KIND == AOTK_Q6_K) {
            const uint2 lo = j < 4 ? cur.q[j] : cur.q2[j - 4];
            const int quarter = j & 3, sh = 2 * quarter;
            const uint32_t n0 = quarter >= 2 ? (lo.x >> 4) & 0x0F0F0F0Fu : lo.x & 0x0F0F0F0Fu;
            const uint32_t n1 = quarter >= 2 ? (lo.y >> 4) & 0x0F0F0F0Fu : lo.y & 0x0F0F0F0Fu;
            const uint32_t v0 = n0 | (((cur.h6[j].x >> sh) & 0x03030303u) << 4);
            const uint32_t v1 = n1 | (((cur.h6[j].y >> sh) & 0x03030303u) << 4);
            // q - 32 per byte (values 0..63, no borrow between bytes)
            w0 = (v0 | 0x80808080u) - 0x20202020u;
            w0 ^= 0x80808080u;
            w1 = (v1 | 0x80808080u) - 0x20202020u;
            w1 ^= 0x80808080u;
        } else {
            const uint2 qb = cur.q[j >> 1];
            const int hi = j & 1;
            w0 = hi ? (qb.x >> 4) & 0x0F0F0F0Fu : qb.x & 0x0F0F0F0Fu;
            w1 = hi ? (qb.y >> 4) & 0x0F0F0F0Fu : qb.y & 0x0F0F0F0Fu;
            if (KIND == AOTK_Q5_K) {
                const uint2 hb = cur.q2[j >> 1];
                w0 |= ((hb.x >> j) & 0x01010101u) << 4;
                w1 |= ((hb.y >> j) & 0x01010101u) << 4;
            }
        }
        b.bq[j] = (long)(((unsigned long)w1 << 32) | w0);
    }
    if (KIND == AOTK_Q6_K) {
        b.dd = cur.d6;
        b.dm = 0.0f;
    } else {
        b.dd = f16_to_f32(cur.hdr.x & 0xFFFFu);
        b.dm = f16_to_f32(cur.hdr.x >> 16);
    }
}

// One 16-token tile of a prepared super-block: exact integer dots
// (v_mfma_i32_16x16x32_i8, A = the tile's activation fragments av[j] =
// token r16's values k = 32j + 8q .. +8), the scale products and the f32
// term of the matvec fold (matvec.rs:82-167 per token): term[i] belongs to
// token 4q + i of the tile and the lane's row; yd[i] is that token's Q8_K d.
template <int KIND>
__device__ __forceinline__ void mm_tile(const MmB<KIND> &b, const long (&av)[8], const float (&yd)[4], int q,
                                        float (&term)[4]) {
    int sumi[4] = {0, 0, 0, 0};
    mm_v4i csum = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 8; j++) {
        if (KIND == AOTK_Q6_K) {
            // two 16-value scale groups per step: lanes q < 2 hold group 2j, q >= 2 group 2j+1
            const long b_lo = q < 2 ? b.bq[j] : 0, b_hi = q < 2 ? 0 : b.bq[j];
            mm_v4i c0 = {0, 0, 0, 0}, c1 = {0, 0, 0, 0};
            c0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[j], b_lo, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[j], b_hi, c1, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) sumi[i] += __mul24(b.sc[2 * j], c0[i]) + __mul24(b.sc[2 * j + 1], c1[i]);
        } else {
            mm_v4i c = {0, 0, 0, 0};
            c = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[j], b.bq[j], c, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; i++) sumi[i] += __mul24(b.sc[j], c[i]);
            const long mb = (long)(0x0101010101010101ULL * (unsigned long)b.mn[j]);
            csum = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[j], mb, csum, 0, 0, 0);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (KIND == AOTK_Q6_K) {
            term[i] = (b.dd * yd[i]) * (float)sumi[i];
        } else {
            term[i] = (b.dd * yd[i]) * (float)sumi[i] - (b.dm * yd[i]) * (float)csum[i];
        }
    }
}

// One super-block of the 16 rows of a wave for its tiles of 16 tokens, the
// activations staged in LDS: ys holds the tiles' activation rows of this
// super-block (MM_YS bytes per token), yds their Q8_K scales; term_out[t][i]
// belongs to token 16t + 4q + i of the lane's row.
template <int KIND, int TT>
__device__ __forceinline__ void mm_sb_terms(const MmW<KIND> &cur, const uint8_t *ys, const float *yds, int q, int r16,
                                            int mt, float (&term_out)[TT][4]) {
    MmB<KIND> b;
    mm_prep<KIND>(cur, b);
#pragma unroll
    for (int t = 0; t < TT; t++) {
        if (16 * t >= mt) break;
        const uint8_t *yrow = ys + (16 * t + r16) * MM_YS + 8 * q;
        long av[8];
#pragma unroll
        for (int j = 0; j < 8; j++) av[j] = *(const long *)(yrow + 32 * j);
        const float yd[4] = {yds[16 * t + 4 * q], yds[16 * t + 4 * q + 1], yds[16 * t + 4 * q + 2], yds[16 * t + 4 * q + 3]};
        mm_tile<KIND>(b, av, yd, q, term_out[t]);
    }
}

template <int KIND, int TT>
__global__ __launch_bounds__(256) void k_mm_kq(MvArgs a, int m) {
    constexpr int NT = 16 * TT;  // tokens per block
    __shared__ __align__(16) uint8_t sY[3][NT * MM_YS];
    __shared__ float sD[3][NT];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int q = lane >> 4, r16 = lane & 15;
    const int nb = a.nb;
    const int grow = blockIdx.x * 64 + wave * 16 + r16;  // this lane's weight row
    const int tok0 = blockIdx.y * NT;                    // the block's first token
    const int mt = min(NT, m - tok0);                    // tokens of this block
    const bool row_ok = grow < a.total_rows;
    int local;
    const int sg = seg_of(a, row_ok ? grow : 0, local);
    const size_t rowb = (size_t)nb * KqGeom<KIND>::RB;
    const uint8_t *rowp = seg_sel(sg, a.w[0], a.w[1], a.w[2]) + (size_t)local * rowb;
    const uint16_t *drow = KIND == AOTK_Q6_K ? (const uint16_t *)seg_sel(sg, a.w1[0], a.w1[1], a.w1[2]) + (size_t)local * nb : nullptr;

    // activation staging: NT tokens x 256 bytes + d of super-block sb, two
    // super-blocks ahead (register sets r0 / r1, LDS ring of 3)
    struct Stg {
        uint4 v[TT];
        float d;
    };
    auto stage_load = [&](Stg &r, int sb) {
#pragma unroll
        for (int k = 0; k < TT; k++) {
            const int idx = tid + 256 * k;  // NT tokens x 16 uint4
            const int tk = idx >> 4, c = idx & 15;
            r.v[k] = tk < mt ? *(const uint4 *)(a.xq + (size_t)(tok0 + tk) * a.cols + (size_t)sb * 256 + 16 * c) : make_uint4(0, 0, 0, 0);
        }
        r.d = (tid < mt) ? a.xd[(size_t)(tok0 + tid) * nb + sb] : 0.0f;
    };
    auto stage_store = [&](const Stg &r, int buf) {
#pragma unroll
        for (int k = 0; k < TT; k++) {
            const int idx = tid + 256 * k;
            const int tk = idx >> 4, c = idx & 15;
            *(uint4 *)(sY[buf] + tk * MM_YS + 16 * c) = r.v[k];
        }
        if (tid < NT) sD[buf][tid] = r.d;
    };

    float acc[TT][4];
#pragma unroll
    for (int t = 0; t < TT; t++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[t][i] = 0.0f;

    MmW<KIND> cur, nxt, nx2;
    Stg r0, r1;
    mm_load<KIND>(cur, rowp, drow, 0, nb, q);
    stage_load(r0, 0);
    stage_store(r0, 0);
    if (nb > 1) {
        mm_load<KIND>(nxt, rowp, drow, 1, nb, q);
        stage_load(r1, 1);
    }
    __syncthreads();
    for (int sb = 0; sb < nb; sb++) {
        const int buf = sb % 3;
        if (sb + 2 < nb) {
            mm_load<KIND>(nx2, rowp, drow, sb + 2, nb, q);
            stage_load(r0, sb + 2);
        }
        float term[TT][4];
        mm_sb_terms<KIND, TT>(cur, sY[buf], sD[buf], q, r16, mt, term);
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (16 * t < mt) acc[t][i] = acc[t][i] + term[t][i];
        if (sb + 1 < nb) stage_store(r1, (sb + 1) % 3);
        __syncthreads();
        cur = nxt;
        nxt = nx2;
        r1 = r0;
    }
    if (row_ok) {
#pragma unroll
        for (int t = 0; t < TT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tk = 16 * t + 4 * q + i;
                if (tk < mt) store_row(a, grow, tok0 + tk, acc[t][i]);
            }
    }
}

// Prompt matmul for matrices of few rows (the grid of k_mm_kq would leave
// CUs idle): the 4 waves of a block share 16 rows and 16*TT tokens and take
// the super-blocks in turn (wave w: w, w + 4, ...), each staging its
// super-block's activations in its own LDS buffers (the next one two steps
// ahead in registers). After every round of 4 super-blocks the terms meet in
// LDS and wave t adds tile t's in super-block order, so the fold is the
// matvec's (bit-identical to m matvecs) while each wave's dependent chain is
// nb/4 super-blocks long and the grid has 4x the waves.
template <int KIND, int TT>
__global__ __launch_bounds__(256) void k_mm_ks(MvArgs a, int m) {
    constexpr int NT = 16 * TT;
    constexpr int SV = NT / 4;  // uint4 per lane of one super-block's staging
    __shared__ __align__(16) uint8_t sY[4][2][NT * MM_YS];
    __shared__ float sD[4][2][NT];
    __shared__ float sT[2][4][TT][4][64];  // [round parity][slot][tile][i][lane]
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, r16 = lane & 15;
    const int nb = a.nb;
    const int grow = blockIdx.x * 16 + r16;
    const int tok0 = blockIdx.y * NT;
    const int mt = min(NT, m - tok0);
    const bool row_ok = grow < a.total_rows;
    int local;
    const int sg = seg_of(a, row_ok ? grow : 0, local);
    const uint8_t *rowp = seg_sel(sg, a.w[0], a.w[1], a.w[2]) + (size_t)local * nb * KqGeom<KIND>::RB;
    const uint16_t *drow = KIND == AOTK_Q6_K ? (const uint16_t *)seg_sel(sg, a.w1[0], a.w1[1], a.w1[2]) + (size_t)local * nb : nullptr;
    struct Stg {
        uint4 v[SV];
        float d;
    };
    auto stage_load = [&](Stg &r, int sb) {
#pragma unroll
        for (int k = 0; k < SV; k++) {
            const int idx = lane + 64 * k;  // NT tokens x 16 uint4
            const int tk = idx >> 4, c = idx & 15;
            r.v[k] = tk < mt ? *(const uint4 *)(a.xq + (size_t)(tok0 + tk) * a.cols + (size_t)sb * 256 + 16 * c) : make_uint4(0, 0, 0, 0);
        }
        r.d = lane < mt ? a.xd[(size_t)(tok0 + lane) * nb + sb] : 0.0f;
    };
    auto stage_store = [&](const Stg &r, int buf) {
#pragma unroll
        for (int k = 0; k < SV; k++) {
            const int idx = lane + 64 * k;
            *(uint4 *)(sY[wave][buf] + (idx >> 4) * MM_YS + 16 * (idx & 15)) = r.v[k];
        }
        if (lane < NT) sD[wave][buf][lane] = r.d;
    };
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // waves < TT: tile `wave`
    const int rounds = (nb + 3) / 4;
    MmW<KIND> cur, nxt;
    Stg r1;
    if (wave < nb) {
        mm_load<KIND>(cur, rowp, drow, wave, nb, q);
        Stg r0;
        stage_load(r0, wave);
        stage_store(r0, 0);
        if (wave + 4 < nb) {
            mm_load<KIND>(nxt, rowp, drow, wave + 4, nb, q);
            stage_load(r1, wave + 4);
        }
    }
    wave_lds_sync();
    for (int r = 0; r < rounds; r++) {
        const int sb = 4 * r + wave;
        if (sb < nb) {
            const int buf = r & 1;
            float term[TT][4];
            mm_sb_terms<KIND, TT>(cur, sY[wave][buf], sD[wave][buf], q, r16, mt, term);
#pragma unroll
            for (int t = 0; t < TT; t++)
#pragma unroll
                for (int i = 0; i < 4; i++) sT[r & 1][wave][t][i][lane] = term[t][i];
            if (sb + 4 < nb) {
                stage_store(r1, buf ^ 1);
                cur = nxt;
                if (sb + 8 < nb) {
                    mm_load<KIND>(nxt, rowp, drow, sb + 8, nb, q);
                    stage_load(r1, sb + 8);
                }
            }
        }
        __syncthreads();
        if (wave < TT) {
            const int n = min(4, nb - 4 * r);
            for (int slot = 0; slot < n; slot++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i] = acc[i] + sT[r & 1][slot][wave][i][lane];
        }
    }
    if (wave < TT && row_ok) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int tk = 16 * wave + 4 * q + i;
            if (tk < mt) store_row(a, grow, tok0 + tk, acc[i]);
        }
    }
}

// Prompt matmul, all tokens (m <= 64) of 16 weight rows per block, the
// super-blocks split over the block's W waves (wave w: w, w + W, ...). The
// activation operands come straight from global memory in the tiled order of
// ActQ8K::qt (16-byte loads, 1 KB contiguous per wave load; the batch stays
// in L2), all token tiles of a super-block issued at once, and the wave's
// next super-block's weights are loaded a whole super-block ahead; the Q8_K
// scales of the batch are staged once per block in LDS, transposed to
// [super-block][token]. Per round of W super-blocks each wave leaves its
// terms in LDS and wave t (t < tiles) adds those of token tile t in
// super-block order, so every output is the matvec's fold (bit-identical to
// m matvecs). Tokens past m in the last tile compute on whatever the tiled
// copy holds there (matrix-core rows are independent) and are not stored.
constexpr int MMX_MAX_NB = 64;

// A operands of token tiles t0, t0 + 1 of super-block sb from the tiled
// copy: lane l's 16 bytes of step pair p at p*1024 + 16l.
__device__ __forceinline__ void mmx_load2(uint4 (&at)[2][4], const int8_t *xt, int sb, int t0, int ntiles,
                                          size_t tile_stride, int lane) {
    const uint8_t *ab = (const uint8_t *)xt + (size_t)sb * 4096 + 16 * lane;
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const int t = min(t0 + u, ntiles - 1);  // past the batch: the last tile again (never folded)
#pragma unroll
        for (int p = 0; p < 4; p++) at[u][p] = *(const uint4 *)(ab + t * tile_stride + p * 1024);
    }
}

// Terms of two token tiles at once (their matrix-core chains interleaved,
// no branches between them) into the wave's LDS slot: the same arithmetic
// as mm_tile per tile. Tiles at or past the batch's last compute on the last
// tile's operands and are never folded.
template <int KIND>
__device__ __forceinline__ void mmx_tiles2(const MmB<KIND> &b, const uint4 (&at)[2][4], const float *sD, int sb, int t0,
                                           int q, int lane, float (*slot)[64][4]) {
    long av[2][8];
#pragma unroll
    for (int u = 0; u < 2; u++)
#pragma unroll
        for (int p = 0; p < 4; p++) {
            av[u][2 * p] = (long)(((unsigned long)at[u][p].y << 32) | at[u][p].x);
            av[u][2 * p + 1] = (long)(((unsigned long)at[u][p].w << 32) | at[u][p].z);
        }
    int sumi[2][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
    mm_v4i csum[2] = {{0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
    for (int j = 0; j < 8; j++) {
        if (KIND == AOTK_Q6_K) {
            const long b_lo = q < 2 ? b.bq[j] : 0, b_hi = q < 2 ? 0 : b.bq[j];
            mm_v4i c0[2], c1[2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const mm_v4i z = {0, 0, 0, 0};
                c0[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[u][j], b_lo, z, 0, 0, 0);
                c1[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[u][j], b_hi, z, 0, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < 2; u++)
#pragma unroll
                for (int i = 0; i < 4; i++) sumi[u][i] += __mul24(b.sc[2 * j], c0[u][i]) + __mul24(b.sc[2 * j + 1], c1[u][i]);
        } else {
            const long mb = (long)(0x0101010101010101ULL * (unsigned long)b.mn[j]);
            mm_v4i c[2];
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const mm_v4i z = {0, 0, 0, 0};
                c[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[u][j], b.bq[j], z, 0, 0, 0);
                csum[u] = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[u][j], mb, csum[u], 0, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < 2; u++)
#pragma unroll
                for (int i = 0; i < 4; i++) sumi[u][i] += __mul24(b.sc[j], c[u][i]);
        }
    }
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const float4 y4 = *(const float4 *)&sD[sb * 64 + 16 * (t0 + u) + 4 * q];
        const float yd[4] = {y4.x, y4.y, y4.z, y4.w};
        float term[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if (KIND == AOTK_Q6_K) term[i] = (b.dd * yd[i]) * (float)sumi[u][i];
            else term[i] = (b.dd * yd[i]) * (float)sumi[u][i] - (b.dm * yd[i]) * (float)csum[u][i];
        }
        *(float4 *)slot[t0 + u][lane] = make_float4(term[0], term[1], term[2], term[3]);
    }
}

// Q4_K on the K = 64 matrix cores with the sub-block scales folded into
// the B operand. Every 6-bit scale is split into two 3-bit parts s_p (the
// quants are <= 15, so q * s_p <= 105): each part's pre-scaled quants are
// exact signed bytes, and v_mfma_i32_16x16x64_i8 of them against the
// activations sums a super-block in four steps. The scaled integer sum of
// the super-block is then C_0 + 8 * C_1, exactly the sum of
// sc_j * (dot of sub-block j) that the matvec forms. The mins term keeps
// its own product against the mins broadcast per sub-block. Lane l's 16
// bytes of step pair J (values 64J + 8q .. +8 and 64J + 32 + 8q .. +8,
// q = l / 16) are the A operand as the tiled copy holds it; B holds the
// same values of the lane's row. (Q5_K the same way needs three 2-bit
// parts and measured 4% slower than the per-sub-block products.)
struct MmP {
    mm_v4i bp[2][4];  // [scale part][step pair J]
    uint32_t mn[8];   // the mins of the sub-blocks, each broadcast to 4 bytes
    float dd, dm;
};

typedef unsigned short mm_u16x2 __attribute__((ext_vector_type(2)));
// Byte-wise product of four bytes by s (every product below 128, so no
// byte carries into the next): two 16-bit lanes of one packed multiply.
__device__ __forceinline__ int mm_bmul(uint32_t w, uint32_t s) {
    const mm_u16x2 a = __builtin_bit_cast(mm_u16x2, w), b = {(unsigned short)s, (unsigned short)s};
    return (int)__builtin_bit_cast(uint32_t, a * b);
}

__device__ __forceinline__ void mm_prep64(const MmW<AOTK_Q4_K> &cur, MmP &b) {
    int sc[8], mn[8];
#pragma unroll
    for (int j = 0; j < 8; j++) scale_min_k4(j, cur.hdr.y, cur.hdr.z, cur.hdr.w, sc[j], mn[j]);
#pragma unroll
    for (int J = 0; J < 4; J++) {
        const uint2 qb = cur.q[J];
        const uint32_t w[4] = {qb.x & 0x0F0F0F0Fu, qb.y & 0x0F0F0F0Fu, (qb.x >> 4) & 0x0F0F0F0Fu, (qb.y >> 4) & 0x0F0F0F0Fu};
#pragma unroll
        for (int pt = 0; pt < 2; pt++) {
            const uint32_t sa = ((uint32_t)sc[2 * J] >> (3 * pt)) & 7u, sb = ((uint32_t)sc[2 * J + 1] >> (3 * pt)) & 7u;
            b.bp[pt][J] = mm_v4i{mm_bmul(w[0], sa), mm_bmul(w[1], sa), mm_bmul(w[2], sb), mm_bmul(w[3], sb)};
        }
        b.mn[2 * J] = (uint32_t)mn[2 * J] * 0x01010101u;
        b.mn[2 * J + 1] = (uint32_t)mn[2 * J + 1] * 0x01010101u;
    }
    b.dd = f16_to_f32(cur.hdr.x & 0xFFFFu);
    b.dm = f16_to_f32(cur.hdr.x >> 16);
}

// Terms of two token tiles from pre-scaled operands (see MmP), the same f32
// term per (row, token) as mm_tile.
__device__ __forceinline__ void mmx_tiles2_64(const MmP &b, const uint4 (&at)[2][4], const float *sD, int sb, int t0, int q,
                                              int lane, float (*slot)[64][4]) {
    mm_v4i c[2][2], cm[2];
#pragma unroll
    for (int u = 0; u < 2; u++) cm[u] = c[u][0] = c[u][1] = mm_v4i{0, 0, 0, 0};
#pragma unroll
    for (int J = 0; J < 4; J++)
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const mm_v4i a = __builtin_bit_cast(mm_v4i, at[u][J]);
            const mm_v4i bm = {(int)b.mn[2 * J], (int)b.mn[2 * J], (int)b.mn[2 * J + 1], (int)b.mn[2 * J + 1]};
            c[u][0] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b.bp[0][J], c[u][0], 0, 0, 0);
            c[u][1] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b.bp[1][J], c[u][1], 0, 0, 0);
            cm[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bm, cm[u], 0, 0, 0);
        }
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const float4 y4 = *(const float4 *)&sD[sb * 64 + 16 * (t0 + u) + 4 * q];
        const float yd[4] = {y4.x, y4.y, y4.z, y4.w};
        float term[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int sumi = c[u][0][i] + (c[u][1][i] << 3);
            term[i] = (b.dd * yd[i]) * (float)sumi - (b.dm * yd[i]) * (float)cm[u][i];
        }
        *(float4 *)slot[t0 + u][lane] = make_float4(term[0], term[1], term[2], term[3]);
    }
}

// The 16-row groups g0, g0 + gs, ... (< the matrix's groups) of one matrix
// for the block (see k_mm_kx); sD holds the batch's Q8_K d as
// [super-block][token], staged by the caller.
template <int KIND, int W>
__device__ __forceinline__ void mm_kx_body(const MvArgs &a, int m, int g0, int gs, const float *sD, float (*sT)[W][4][64][4]) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, r16 = lane & 15;
    const int nb = a.nb;
    const int mt = min(64, m);
    const int ntiles = (mt + 15) / 16;
    const int ngroups = (a.total_rows + 15) / 16;
    const int rounds = (nb + W - 1) / W;
    const size_t tile_stride = (size_t)nb * 4096;
    // the wave's items: (row group g, super-block sb)
    auto rows_of = [&](int g, const uint8_t *&rowp, const uint16_t *&drow) {
        const int grow = g * 16 + r16;
        int local;
        const int sg = seg_of(a, grow < a.total_rows ? grow : 0, local);
        rowp = seg_sel(sg, a.w[0], a.w[1], a.w[2]) + (size_t)local * nb * KqGeom<KIND>::RB;
        drow = KIND == AOTK_Q6_K ? (const uint16_t *)seg_sel(sg, a.w1[0], a.w1[1], a.w1[2]) + (size_t)local * nb : nullptr;
    };
    if (g0 >= ngroups) return;  // (block-uniform)
    const uint8_t *rowp, *rown;
    const uint16_t *drow, *drown;
    int g = g0;
    rows_of(g, rowp, drow);
    MmW<KIND> cur, nxt;
    if (wave < nb) mm_load<KIND>(cur, rowp, drow, wave, nb, q);
    __syncthreads();  // (the staged d: the first weights are in flight meanwhile)
    int par = 0;
    for (; g < ngroups; g += gs) {
        const int gn = g + gs;
        if (gn < ngroups) rows_of(gn, rown, drown);
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // waves < ntiles: tile `wave`
        for (int r = 0; r < rounds; r++, par ^= 1) {
            const int sb = r * W + wave;
            if (sb < nb) {
                // the next item's weights: the next round of this group, or the first of the next group
                if (sb + W < nb) mm_load<KIND>(nxt, rowp, drow, sb + W, nb, q);
                else if (gn < ngroups) mm_load<KIND>(nxt, rown, drown, wave, nb, q);
                uint4 at[2][4];
                mmx_load2(at, a.xt, sb, 0, ntiles, tile_stride, lane);
                if constexpr (KIND != AOTK_Q4_K) {
                    MmB<KIND> b;
                    mm_prep<KIND>(cur, b);
                    mmx_tiles2<KIND>(b, at, sD, sb, 0, q, lane, sT[par][wave]);
                    if (ntiles > 2) {
                        mmx_load2(at, a.xt, sb, 2, ntiles, tile_stride, lane);
                        mmx_tiles2<KIND>(b, at, sD, sb, 2, q, lane, sT[par][wave]);
                    }
                } else {
                    MmP b;
                    mm_prep64(cur, b);
                    mmx_tiles2_64(b, at, sD, sb, 0, q, lane, sT[par][wave]);
                    if (ntiles > 2) {
                        mmx_load2(at, a.xt, sb, 2, ntiles, tile_stride, lane);
                        mmx_tiles2_64(b, at, sD, sb, 2, q, lane, sT[par][wave]);
                    }
                }
                cur = nxt;
            }
            __syncthreads();
            if (wave < ntiles) {
                const int n = min(W, nb - r * W);
                for (int slot = 0; slot < n; slot++) {
                    const float4 v = *(const float4 *)sT[par][slot][wave][lane];
                    acc[0] = acc[0] + v.x;
                    acc[1] = acc[1] + v.y;
                    acc[2] = acc[2] + v.z;
                    acc[3] = acc[3] + v.w;
                }
            }
        }
        const int grow = g * 16 + r16;
        if (wave < ntiles && grow < a.total_rows) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tk = 16 * wave + 4 * q + i;
                if (tk < mt) store_row(a, grow, tk, acc[i]);
            }
        }
        rowp = rown;
        drow = drown;
    }
    __syncthreads();  // the caller may reuse sT
}

// The batch's Q8_K d into LDS as [super-block][token].
template <int NT>
__device__ __forceinline__ void mm_kx_stage_d(const MvArgs &a, int m, float *sD) {
    // every load first (unconditional: indices past the end re-read the
    // last), then the stores: one wait instead of one per element
    constexpr int PER = (MMX_MAX_NB * 64 + NT - 1) / NT;
    const int mt = min(64, m), nb = a.nb, tot = mt * nb;
    float v[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) v[j] = a.xd[min((int)threadIdx.x + j * NT, tot - 1)];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int idx = threadIdx.x + j * NT;
        if (idx < tot) {
            const int tk = idx / nb, sb = idx - tk * nb;
            sD[sb * 64 + tk] = v[j];
        }
    }
}

template <int KIND, int W>
__global__ __launch_bounds__(64 * W) void k_mm_kx(MvArgs a, int m) {
    __shared__ __align__(16) float sD[MMX_MAX_NB * 64];    // [super-block][token]
    __shared__ __align__(16) float sT[2][W][4][64][4];     // [round parity][slot][tile][lane][i]
    mm_kx_stage_d<64 * W>(a, m, sD);
    mm_kx_body<KIND, W>(a, m, blockIdx.x, gridDim.x, sD, sT);
}

// Two matrices of different kinds on the same batch in one persistent
// launch (the prompt's q/k and v): the grid walks the groups of `a`, then
// those of `b`, as one list of items, so that the second matrix fills the
// blocks the first leaves idle in its last round. Both share the staged d.
template <int KA, int KB, int W>
__global__ __launch_bounds__(64 * W) void k_mm_kx2(MvArgs a, MvArgs b, int m) {
    __shared__ __align__(16) float sD[MMX_MAX_NB * 64];
    __shared__ __align__(16) float sT[2][W][4][64][4];
    mm_kx_stage_d<64 * W>(a, m, sD);
    const int G = gridDim.x, ga = (a.total_rows + 15) / 16;
    mm_kx_body<KA, W>(a, m, blockIdx.x, G, sD, sT);
    // item i >= ga of the combined list is group i - ga of b; this block's
    // first such item
    const int first = (int)blockIdx.x + ((ga - (int)blockIdx.x + G - 1) / G) * G;  // smallest i >= ga, i = blockIdx.x (mod G)
    mm_kx_body<KB, W>(b, m, first - ga, G, sD, sT);
}

// ------------------------------------------------------ Q8_0 / Q4_0 / Q5_0
// Wave = 8 rows. Phase A: lanes turn 32 blocks of 2 rows per pass into the 8
// per-lane integer sums P and the scale D = f16(d) * y.d, staged in LDS.
// Phase B: lane (row r, chain l) runs acc_l = fma(D, P_l, acc_l) in block
// order. Then the avx2 horizontal sum.
constexpr int Q80_STEP = 32;

template <int KIND>
__global__ __launch_bounds__(256) void k_mv_q80(MvArgs a) {
    __shared__ float sP[4][8][Q80_STEP][8];
    __shared__ float sD[4][8][Q80_STEP];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int tok = blockIdx.y;
    const int grow0 = (blockIdx.x * 4 + wave) * 8;
    const int nb = a.nb;
    const int8_t *xq = a.xq + (size_t)tok * a.cols;
    const float *xd = a.xd + (size_t)tok * nb;
    float acc = 0.0f;
    const int rb_row = lane >> 3, chain = lane & 7;

    for (int i0 = 0; i0 < nb; i0 += Q80_STEP) {
        for (int pass = 0; pass < 4; pass++) {
            const int rr = 2 * pass + (lane >> 5);
            const int bi = i0 + (lane & 31);
            const int grow = grow0 + rr;
            float P[8];
            float D = 0.0f;
            for (int l = 0; l < 8; l++) P[l] = 0.0f;
            if (grow < a.total_rows && bi < nb) {
                int local;
                int s = seg_of(a, grow, local);
                const size_t blk = (size_t)local * nb + bi;
                const uint4 y0 = *(const uint4 *)(xq + (size_t)bi * 32);
                const uint4 y1 = *(const uint4 *)(xq + (size_t)bi * 32 + 16);
                const uint32_t yw[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
                const float dw = f16_to_f32(((const uint16_t *)seg_sel(s, a.w1[0], a.w1[1], a.w1[2]))[blk]);
                D = dw * xd[bi];
                if (KIND == AOTK_Q8_0) {
                    const uint4 w0 = *(const uint4 *)(seg_sel(s, a.w[0], a.w[1], a.w[2]) + blk * 32);
                    const uint4 w1 = *(const uint4 *)(seg_sel(s, a.w[0], a.w[1], a.w[2]) + blk * 32 + 16);
                    const uint32_t ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
                    for (int l = 0; l < 8; l++) P[l] = (float)dot4(ww[l], yw[l], 0);
                } else {
                    const uint4 w0 = *(const uint4 *)(seg_sel(s, a.w[0], a.w[1], a.w[2]) + blk * 16);
                    const uint32_t nw[4] = {w0.x, w0.y, w0.z, w0.w};
                    uint32_t qh = 0;
                    if (KIND == AOTK_Q5_0) qh = ((const uint32_t *)seg_sel(s, a.w2[0], a.w2[1], a.w2[2]))[blk];
                    for (int l = 0; l < 8; l++) {
                        uint32_t v = l < 4 ? (nw[l] & 0x0F0F0F0Fu) : ((nw[l - 4] >> 4) & 0x0F0F0F0Fu);
                        int off;
                        if (KIND == AOTK_Q5_0) {
                            uint32_t b4 = (qh >> (4 * l)) & 0xFu;
                            uint32_t spread = (b4 & 1u) | ((b4 & 2u) << 7) | ((b4 & 4u) << 14) | ((b4 & 8u) << 21);
                            v |= spread << 4;
                            off = dot4(0xF0F0F0F0u, yw[l], 0);  // -16 * sum(y)
                        } else {
                            off = dot4(0xF8F8F8F8u, yw[l], 0);  // -8 * sum(y)
                        }
                        P[l] = (float)dot4(v, yw[l], off);
                    }
                }
            }
            float *dst = &sP[wave][rr][lane & 31][0];
            *(float4 *)dst = make_float4(P[0], P[1], P[2], P[3]);
            *(float4 *)(dst + 4) = make_float4(P[4], P[5], P[6], P[7]);
            sD[wave][rr][lane & 31] = D;
        }
        __syncthreads();
        const int nstep = nb - i0 < Q80_STEP ? nb - i0 : Q80_STEP;
        for (int ii = 0; ii < nstep; ii++) acc = fmaf(sD[wave][rb_row][ii], sP[wave][rb_row][ii][chain], acc);
        __syncthreads();
    }
    // ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7))  (simd_avx2.rs:27-34)
    float t = acc + shfl_xor(acc, 4);
    float u = t + shfl_xor(t, 2);
    float v = u + shfl_xor(u, 1);
    const int grow = grow0 + rb_row;
    if (chain == 0 && grow < a.total_rows) store_row(a, grow, tok, v);
}

// Q8_0 / Q4_0 / Q5_0, inputs of up to Q8B_MAX_COLS: wave = Q8B_R rows; lane
// = block index within a step of 64 blocks. Phase A: each lane forms, for
// each of the wave's rows, the 8 per-lane integer sums P_l of its block and
// the scale D = f16(d) * y.d (the activation is staged in LDS per block of
// 256 threads), written to LDS; phase B: lane (row r, chain l) runs
// acc_l = fma(D, P_l, acc_l) over the step's blocks in order. The next
// step's weights are loaded during phase B. Then the avx2 horizontal sum.
// Phase B runs on 8 * Q8B_R lanes (16 of the 64 with two rows per wave);
// the others idle there, which measured cheaper than the larger phase A
// that more rows per wave need.
constexpr int Q8B_R = 2;  // measured: 2 rows per wave beat 4 (Q8_0 14336x4096 14.5 against 17.7 us) and 1
constexpr int Q8B_MAX_COLS = 16384;
constexpr int Q8B_CS = 64 + 4;  // floats per (row, chain) line of the P buffer: chain-major, padded
// the block of a Q8_0 step that lane l holds after the half swap
__device__ __forceinline__ int q8_slot(int l) { return (l & 1) * 32 + (l >> 1); }

template <int KIND>
struct Q8bW {
    uint4 w0, w1;  // Q8_0: 32 quants; Q4_0/Q5_0: w0 = 16 nibble bytes
    uint32_t qh;   // Q5_0
    uint16_t d;
};

template <int KIND, bool XQ = false, bool RUNS = KIND == AOTK_Q8_0>
__global__ __launch_bounds__(256) void k_mv_q8b(MvArgs a) {
    constexpr int R = Q8B_R;
    // the activation (cols int8 quants, then cols / 32 scales), sized by the
    // launch so that short rows leave LDS for more blocks per CU
    extern __shared__ __align__(16) int8_t sy[];
    float *syd = (float *)(sy + a.cols);
    __shared__ __align__(16) float sP[4][R][8][Q8B_CS];
    __shared__ __align__(16) float sD[4][R][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tok = blockIdx.y;
    const int nb = a.nb;
    // weights of this wave's rows (rows past the end read row 0)
    const uint8_t *wq[R];
    const uint16_t *wd[R];
    const uint32_t *wh[R];
    const int grow0 = (blockIdx.x * 4 + wave) * R;
#pragma unroll
    for (int r = 0; r < R; r++) {
        int local;
        const int sg = seg_of(a, grow0 + r < a.total_rows ? grow0 + r : 0, local);
        constexpr int QB = KIND == AOTK_Q8_0 ? 32 : 16;
        wq[r] = seg_sel(sg, a.w[0], a.w[1], a.w[2]) + (size_t)local * nb * QB;
        wd[r] = (const uint16_t *)seg_sel(sg, a.w1[0], a.w1[1], a.w1[2]) + (size_t)local * nb;
        wh[r] = KIND == AOTK_Q5_0 ? (const uint32_t *)seg_sel(sg, a.w2[0], a.w2[1], a.w2[2]) + (size_t)local * nb : nullptr;
    }
    // Q8_0 with RUNS: the step's 64 blocks of 32 bytes are read as two
    // contiguous 1 KB runs with the nontemporal hint, lane l taking half
    // l & 1 of block l >> 1 (w0) and of block 32 + (l >> 1) (w1), so that
    // each load instruction covers whole cache lines (nontemporal loads of
    // lines split over two instructions fetched them twice); the lane pairs
    // then swap halves (step), and lane l ends up with block q8_slot(l).
    // Measured: Qwen3 decode 234 -> 236 tok/s, Q8_0 4096x14336 14.2 -> 13.7
    // us; the lm-head shape (128256 rows) ran 96 -> 102 us with it and is
    // launched without (RUNS = false: lane l reads block l with plain loads).
    auto load = [&](Q8bW<KIND> (&w)[R], int c0) {
        const int b = min(c0 + lane, nb - 1);
        const size_t h0 = (size_t)min(c0 + (lane >> 1), nb - 1) * 32 + (lane & 1) * 16;
        const size_t h1 = (size_t)min(c0 + 32 + (lane >> 1), nb - 1) * 32 + (lane & 1) * 16;
        const int bd = min(c0 + q8_slot(lane), nb - 1);
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (KIND == AOTK_Q8_0 && RUNS) {
                w[r].w0 = ld_weights<true>(wq[r] + h0);
                w[r].w1 = ld_weights<true>(wq[r] + h1);
                w[r].d = wd[r][bd];
            } else if (KIND == AOTK_Q8_0) {
                w[r].w0 = *(const uint4 *)(wq[r] + (size_t)b * 32);
                w[r].w1 = *(const uint4 *)(wq[r] + (size_t)b * 32 + 16);
                w[r].d = wd[r][b];
            } else {
                w[r].w0 = ld_weights<true>(wq[r] + (size_t)b * 16);
                if (KIND == AOTK_Q5_0) w[r].qh = wh[r][b];
                w[r].d = wd[r][b];
            }
        }
    };
    // the activation's loads first (cols <= 16384: at most 4 quads and one
    // scale per thread, indices past the end re-read the last), then the
    // first two steps' weights: the wait for the activation leaves those in
    // flight
    Q8bW<KIND> cur[R], nxt[R];
    if constexpr (!XQ) {
        const uint4 *xq = (const uint4 *)(a.xq + (size_t)tok * a.cols);
        const int nq = (int)(a.cols / 16);
        uint4 xv[4];
#pragma unroll
        for (int k = 0; k < 4; k++) xv[k] = xq[min(tid + 256 * k, nq - 1)];
        float xdv[2];
#pragma unroll
        for (int k = 0; k < 2; k++) xdv[k] = a.xd[(size_t)tok * nb + min(tid + 256 * k, nb - 1)];
        load(cur, 0);
        load(nxt, 64);
        // (unconditional stores: past the end they repeat the last element's
        // value at its own place, which keeps the loads above unconditional too)
#pragma unroll
        for (int k = 0; k < 4; k++) ((uint4 *)sy)[min(tid + 256 * k, nq - 1)] = xv[k];
#pragma unroll
        for (int k = 0; k < 2; k++) syd[min(tid + 256 * k, nb - 1)] = xdv[k];
    } else {
        // one token, the f32 input (a.xq_src, cols % 256 == 0) quantized to
        // Q8_0 here by every block (the quantizer of k_quant_f32): wave w
        // takes the 256-value groups w, w + 4, ..., four loads in flight
        const int ng = (int)(a.cols / 256);
        float4 xf[4];
#pragma unroll
        for (int k = 0; k < 4; k++) xf[k] = ((const float4 *)(a.xq_src + (size_t)min(wave + 4 * k, ng - 1) * 256))[lane];
        load(cur, 0);
        load(nxt, 64);
        // the input's loads stay ahead of the weights' and its quantization
        // after them (no code motion across this point): the quantizer then
        // waits for the input only, with the weights in flight
#pragma unroll
        for (int k = 0; k < 4; k++) pin_after_loads(xf[k]);
        // (the first four groups straight from xf, not through a select
        // with a load: that load would issue after the weights' and its wait
        // would wait for them)
        for (int g0 = wave; g0 < ng; g0 += 16) {
            float4 v4[4];
            if (g0 == wave) {
#pragma unroll
                for (int k = 0; k < 4; k++) v4[k] = xf[k];
            } else {
#pragma unroll
                for (int k = 0; k < 4; k++) v4[k] = ((const float4 *)(a.xq_src + (size_t)min(g0 + 4 * k, ng - 1) * 256))[lane];
            }
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int g = g0 + 4 * k;
                if (g >= ng) break;
                const float v[4] = {v4[k].x, v4[k].y, v4[k].z, v4[k].w};
                int qv[4];
                float d;
                ((uint32_t *)(sy + g * 256))[lane] = q80_lane(v, qv, d);
                if ((lane & 7) == 0) syd[g * 8 + (lane >> 3)] = d;
            }
        }
    }
    __syncthreads();
    const int rr = lane >> 3, chain = lane & 7;
    float acc = 0.0f;
    // one step of 64 blocks: phase A (the integer sums and scales into LDS),
    // phase B (the chains)
    auto step = [&](const Q8bW<KIND> (&w_in)[R], int c0) {
        // phase A
        const int slot = KIND == AOTK_Q8_0 && RUNS ? q8_slot(lane) : lane;
        const int b = c0 + slot;
        Q8bW<KIND> w[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            w[r] = w_in[r];
            if (KIND == AOTK_Q8_0 && RUNS) {
                // even lanes send their half of block 32 + l/2, odd lanes
                // theirs of block l/2 (full exec mask: the swap precedes
                // every branch)
                const bool odd = lane & 1;
                const uint4 snd = odd ? w_in[r].w0 : w_in[r].w1;
                const uint4 rcv = make_uint4(dppx_u<DPP_XOR1>(snd.x), dppx_u<DPP_XOR1>(snd.y),
                                             dppx_u<DPP_XOR1>(snd.z), dppx_u<DPP_XOR1>(snd.w));
                w[r].w0 = odd ? rcv : w_in[r].w0;
                w[r].w1 = odd ? w_in[r].w1 : rcv;
            }
        }
        if (b < nb) {
            const uint4 y0 = *(const uint4 *)(sy + b * 32), y1 = *(const uint4 *)(sy + b * 32 + 16);
            const uint32_t yw[8] = {y0.x, y0.y, y0.z, y0.w, y1.x, y1.y, y1.z, y1.w};
            const float yd = syd[b];
            int off[8];
            if (KIND != AOTK_Q8_0)
#pragma unroll
                for (int l = 0; l < 8; l++) off[l] = dot4(KIND == AOTK_Q5_0 ? 0xF0F0F0F0u : 0xF8F8F8F8u, yw[l], 0);
#pragma unroll
            for (int r = 0; r < R; r++) {
                float P[8];
                if (KIND == AOTK_Q8_0) {
                    const uint32_t ww[8] = {w[r].w0.x, w[r].w0.y, w[r].w0.z, w[r].w0.w,
                                            w[r].w1.x, w[r].w1.y, w[r].w1.z, w[r].w1.w};
#pragma unroll
                    for (int l = 0; l < 8; l++) P[l] = (float)dot4(ww[l], yw[l], 0);
                } else {
                    const uint32_t nw[4] = {w[r].w0.x, w[r].w0.y, w[r].w0.z, w[r].w0.w};
#pragma unroll
                    for (int l = 0; l < 8; l++) {
                        uint32_t v = l < 4 ? (nw[l] & 0x0F0F0F0Fu) : ((nw[l - 4] >> 4) & 0x0F0F0F0Fu);
                        if (KIND == AOTK_Q5_0) {
                            const uint32_t b4 = (w[r].qh >> (4 * l)) & 0xFu;
                            const uint32_t spread = (b4 & 1u) | ((b4 & 2u) << 7) | ((b4 & 4u) << 14) | ((b4 & 8u) << 21);
                            v |= spread << 4;
                        }
                        P[l] = (float)dot4(v, yw[l], off[l]);
                    }
                }
#pragma unroll
                for (int l = 0; l < 8; l++) sP[wave][r][l][slot] = P[l];
                sD[wave][r][slot] = f16_to_f32(w[r].d) * yd;
            }
        }
        wave_lds_sync();
        // phase B: block order, one fma chain per (row, lane chain)
        if (rr < R) {
            const int n = nb - c0 < 64 ? nb - c0 : 64;
            // chain-major P and contiguous D: 16-byte reads (D is the same
            // for the row's 8 chains, a broadcast)
            const float *pp = sP[wave][rr][chain];
            const float *dp = sD[wave][rr];
            int i = 0;
            for (; i + 8 <= n; i += 8) {
                const float4 p0 = *(const float4 *)(pp + i), p1 = *(const float4 *)(pp + i + 4);
                const float4 d0 = *(const float4 *)(dp + i), d1 = *(const float4 *)(dp + i + 4);
                acc = fmaf(d0.x, p0.x, acc);
                acc = fmaf(d0.y, p0.y, acc);
                acc = fmaf(d0.z, p0.z, acc);
                acc = fmaf(d0.w, p0.w, acc);
                acc = fmaf(d1.x, p1.x, acc);
                acc = fmaf(d1.y, p1.y, acc);
                acc = fmaf(d1.z, p1.z, acc);
                acc = fmaf(d1.w, p1.w, acc);
            }
            for (; i < n; i++) acc = fmaf(dp[i], pp[i], acc);
        }
        wave_lds_sync();
    };
    // two register sets in turn, no copies; every load is unconditional
    // (steps past the end re-read the last block), so the waits stay exact
    for (int c0 = 0; c0 < nb; c0 += 128) {
        step(cur, c0);
        load(cur, c0 + 128);
        if (c0 + 64 >= nb) break;
        step(nxt, c0 + 64);
        load(nxt, c0 + 192);
    }
    // ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7))  (simd_avx2.rs:27-34)
    const float t = acc + shfl_xor(acc, 4);
    const float u = t + shfl_xor(t, 2);
    const float v = u + shfl_xor(u, 1);
    const int grow = grow0 + rr;
    if (rr < R && chain == 0 && grow < a.total_rows) store_row(a, grow, tok, v);
}

// ------------------------------------------------------- F16 / BF16 / F32
template <int KIND>
__device__ __forceinline__ float wval(const uint8_t *row, size_t i) {
    if (KIND == AOTK_F32) return ((const float *)row)[i];
    uint32_t h = ((const uint16_t *)row)[i];
    if (KIND == AOTK_BF16) return bf16_to_f32(h);
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

template <int KIND>
__global__ __launch_bounds__(256) void k_mv_float(MvArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int tok = blockIdx.y;
    const int r8 = lane >> 3, l = lane & 7;
    const int grow = (blockIdx.x * 4 + wave) * 8 + r8;
    const bool valid = grow < a.total_rows;
    int local;
    const int s = seg_of(a, valid ? grow : 0, local);
    const uint8_t *row = seg_sel(s, a.w[0], a.w[1], a.w[2]) + (size_t)local * a.rb;
    const float *x = a.xf + (size_t)tok * a.cols;
    const size_t n8 = a.cols / 8;
    float acc = 0.0f;
    if (valid) {
        size_t sI = 0;
        for (; sI + 4 <= n8; sI += 4) {
            float w0 = wval<KIND>(row, 8 * sI + l), w1 = wval<KIND>(row, 8 * (sI + 1) + l);
            float w2 = wval<KIND>(row, 8 * (sI + 2) + l), w3 = wval<KIND>(row, 8 * (sI + 3) + l);
            float x0 = x[8 * sI + l], x1 = x[8 * (sI + 1) + l], x2 = x[8 * (sI + 2) + l], x3 = x[8 * (sI + 3) + l];
            acc = fmaf(w0, x0, acc);
            acc = fmaf(w1, x1, acc);
            acc = fmaf(w2, x2, acc);
            acc = fmaf(w3, x3, acc);
        }
        for (; sI < n8; sI++) acc = fmaf(wval<KIND>(row, 8 * sI + l), x[8 * sI + l], acc);
    }
    float t = acc + shfl_xor(acc, 4);
    float u = t + shfl_xor(t, 2);
    float v = u + shfl_xor(u, 1);
    if (l == 0 && valid) {
        for (size_t i = n8 * 8; i < a.cols; i++) v = v + wval<KIND>(row, i) * x[i];
        store_row(a, grow, tok, v);
    }
}

// F16 / BF16 rows of cols % 64 == 0, cols <= MVH_MAX_COLS: the same eight
// chains (chain l takes the elements l, l + 8, l + 16, ... of the row, one
// fmaf each, in order) with wide loads. The 8 lanes of a row load 128
// contiguous bytes per step (lane l: elements 64t + 8l .. + 7, i.e. one
// element of every chain) and an 8x8 transpose of 16-bit values over the
// lanes (three butterfly stages) hands lane l the eight consecutive elements
// of its own chain. The activation sits in LDS chain-major (xs[l][s] =
// x[8s + l]), so lane l reads its eight x values as two 16-byte words.
constexpr int MVH_MAX_COLS = 16128;  // 8 * S floats of LDS stay within 64 KiB

template <int CTRL, int BANKS>
__device__ __forceinline__ uint32_t dpp_upd(uint32_t old, uint32_t src) {
    return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)src, CTRL, 0xF, BANKS, false);
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}

// d: halves c = 0..7 of lane l (element (l, c)); afterwards element (c, l).
// Stage m swaps lane bit m with position bit m where they differ.
__device__ __forceinline__ void transpose8x8_u16(uint32_t d[4], int l) {
    {  // bit 2: dwords 2,3 of lanes 0-3 <-> dwords 0,1 of lanes 4-7. row_shr:4
        // (lane i reads i - 4) written to banks 1,3 (lanes 4-7 of each 8),
        // row_shl:4 (lane i reads i + 4) to banks 0,2.
        const uint32_t n0 = dpp_upd<0x114, 0xA>(d[0], d[2]);
        const uint32_t n1 = dpp_upd<0x114, 0xA>(d[1], d[3]);
        const uint32_t n2 = dpp_upd<0x104, 0x5>(d[2], d[0]);
        const uint32_t n3 = dpp_upd<0x104, 0x5>(d[3], d[1]);
        d[0] = n0; d[1] = n1; d[2] = n2; d[3] = n3;
    }
    {  // bit 1: dwords 1,3 of lanes {0,1} <-> dwords 0,2 of lanes {2,3} (mod 4);
        // quad_perm [0,1,0,1] and [2,3,2,3]
        const bool hi = l & 2;
        const uint32_t a0 = dpp_mov<0x44>(d[1]), a2 = dpp_mov<0x44>(d[3]);
        const uint32_t b1 = dpp_mov<0xEE>(d[0]), b3 = dpp_mov<0xEE>(d[2]);
        if (hi) { d[0] = a0; d[2] = a2; } else { d[1] = b1; d[3] = b3; }
    }
    {  // lane bit 0 <-> position bit 0 (low <-> high halves); byte selectors
        // by lane parity: send the four halves the partner takes packed in
        // two dwords, then put the received ones in place
        const bool hi = l & 1;
        const uint32_t ssend = hi ? 0x05040100u : 0x07060302u;
        const uint32_t srcv0 = hi ? 0x07060100u : 0x01000504u;
        const uint32_t srcv1 = hi ? 0x07060302u : 0x03020504u;
        const uint32_t r0 = dpp_mov<0xB1>(__builtin_amdgcn_perm(d[1], d[0], ssend));  // quad_perm [1,0,3,2]
        const uint32_t r1 = dpp_mov<0xB1>(__builtin_amdgcn_perm(d[3], d[2], ssend));
        d[0] = __builtin_amdgcn_perm(d[0], r0, srcv0);
        d[1] = __builtin_amdgcn_perm(d[1], r0, srcv1);
        d[2] = __builtin_amdgcn_perm(d[2], r1, srcv0);
        d[3] = __builtin_amdgcn_perm(d[3], r1, srcv1);
    }
}

template <int KIND>
__device__ __forceinline__ float half_lo(uint32_t v) {
    if (KIND == AOTK_BF16) return __uint_as_float(v << 16);
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v & 0xFFFF));
}
template <int KIND>
__device__ __forceinline__ float half_hi(uint32_t v) {
    if (KIND == AOTK_BF16) return __uint_as_float(v & 0xFFFF0000u);
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(v >> 16));
}

template <int KIND, int MVH_U>
__global__ __launch_bounds__(256) void k_mv_half(MvArgs a) {
    extern __shared__ float xs[];  // [8][S]
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int tok = blockIdx.y;
    const int r8 = lane >> 3, l = lane & 7;
    const int n8 = (int)(a.cols >> 3);
    const int S = ((n8 + 31) & ~31) + 4;
    const int grow = (blockIdx.x * 4 + wave) * 8 + r8;
    const bool valid = grow < a.total_rows;
    int local;
    const int s = seg_of(a, valid ? grow : 0, local);
    const uint4 *row = (const uint4 *)(seg_sel(s, a.w[0], a.w[1], a.w[2]) + (size_t)(valid ? local : 0) * a.rb) + l;
    const int nt = n8 >> 3;  // 64-element steps (>= 1)
    // The activation goes to LDS chain-major; its first 4096 elements are
    // loaded before the first weights (the wait for them then leaves the
    // weight loads in flight).
    const float4 *x4 = (const float4 *)(a.xf + (size_t)tok * a.cols);
    const int n4 = (int)(a.cols >> 2);
    auto put_x = [&](int i4, const float4 &v) {  // elements 4 i4 .. + 3: chains (4 i4) & 7 .. + 3
        const int i = 4 * i4;
        float *p = xs + (i & 7) * S + (i >> 3);
        p[0] = v.x;
        p[S] = v.y;
        p[2 * S] = v.z;
        p[3 * S] = v.w;
    };
    float4 xv[4];
#pragma unroll
    for (int k = 0; k < 4; k++) xv[k] = x4[min((int)threadIdx.x + 256 * k, n4 - 1)];
    // Loads past the row's end re-read its last step (always in bounds, so
    // every load is unconditional and the waits stay exact).
    auto ld = [&](int t) { return row[8 * min(t, nt - 1)]; };
    uint4 cur[MVH_U], nxt[MVH_U];
#pragma unroll
    for (int u = 0; u < MVH_U; u++) cur[u] = ld(u);
#pragma unroll
    for (int k = 0; k < 4; k++)
        if ((int)threadIdx.x + 256 * k < n4) put_x(threadIdx.x + 256 * k, xv[k]);
    for (int i4 = threadIdx.x + 1024; i4 < n4; i4 += 256) put_x(i4, x4[i4]);
    __syncthreads();
    const float *xl = xs + l * S;
    float acc = 0.0f;
    auto step = [&](const uint4 &w, int t) {
        uint32_t d[4] = {w.x, w.y, w.z, w.w};
        transpose8x8_u16(d, l);
        const float4 xa = *(const float4 *)(xl + 8 * t);
        const float4 xb = *(const float4 *)(xl + 8 * t + 4);
        acc = fmaf(half_lo<KIND>(d[0]), xa.x, acc);
        acc = fmaf(half_hi<KIND>(d[0]), xa.y, acc);
        acc = fmaf(half_lo<KIND>(d[1]), xa.z, acc);
        acc = fmaf(half_hi<KIND>(d[1]), xa.w, acc);
        acc = fmaf(half_lo<KIND>(d[2]), xb.x, acc);
        acc = fmaf(half_hi<KIND>(d[2]), xb.y, acc);
        acc = fmaf(half_lo<KIND>(d[3]), xb.z, acc);
        acc = fmaf(half_hi<KIND>(d[3]), xb.w, acc);
    };
    int t0 = 0;
    for (; t0 + MVH_U <= nt; t0 += MVH_U) {
#pragma unroll
        for (int u = 0; u < MVH_U; u++) nxt[u] = ld(t0 + MVH_U + u);
#pragma unroll
        for (int u = 0; u < MVH_U; u++) step(cur[u], t0 + u);
#pragma unroll
        for (int u = 0; u < MVH_U; u++) cur[u] = nxt[u];
    }
#pragma unroll
    for (int u = 0; u < MVH_U; u++)
        if (t0 + u < nt) step(cur[u], t0 + u);
    // ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7))  (simd_avx2.rs:27-34)
    const float t = acc + shfl_xor(acc, 4);
    const float u = t + shfl_xor(t, 2);
    const float v = u + shfl_xor(u, 1);
    if (l == 0 && valid) store_row(a, grow, tok, v);
}

static bool mv_half_fits(const MvArgs &a) {
    if (a.cols % 64 != 0 || a.cols > (size_t)MVH_MAX_COLS) return false;
    for (int i = 0; i < a.nseg; i++)
        if ((uintptr_t)a.w[i] % 16 != 0) return false;
    return true;
}

// ------------------------------------------- prompt matmul: Q8_0 family, floats
// Batches of 2 or more tokens for the kinds whose reference kernels keep 8
// f32 lanes (dot_*_q8_0 / dot_f16_f32 ..., simd_avx2.rs:58-129, 433-493, and
// their x4 forms, :273-330, bit-identical to the singles). Lane = token (64
// per grid row), wave = MQ_R weight rows, block = 4 waves. A wave's weights
// are the same for all its lanes: scalar loads (s_load), the nibble unpacking
// on the scalar unit. The activation tile of a stage (MQ_BS blocks of 32, or
// 64 float elements, for 64 tokens) is staged in LDS, two stages in turn,
// with the next stage's loads in flight during the current one. Per
// (row, token) the 8 chains run in element order exactly as in the matvec
// kernels, then the avx2 horizontal sum (and, for floats, the scalar tail):
// a batch equals m matvecs bit for bit.
constexpr int MQ_R = 4;  // rows per wave of k_mm_float

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x8_t __attribute__((ext_vector_type(8)));

// A load whose address is the same for every lane of the wave, through the
// scalar data cache (read only).
template <typename T>
__device__ __forceinline__ T uload(const void *p) {
    return *(const __attribute__((address_space(4))) T *)p;
}

// f16 element i of a uniform array of halves (4-byte aligned scalar load).
__device__ __forceinline__ uint32_t uload_half(const uint16_t *base, size_t i) {
    const uintptr_t at = (uintptr_t)(base + i);
    const uint32_t v = uload<uint32_t>((const void *)(at & ~(uintptr_t)3));
    return (at & 2) ? v >> 16 : v & 0xFFFFu;
}

__device__ __forceinline__ float hsum8(const float (&c)[8]) {
    // ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7))  (simd_avx2.rs:27-34)
    return ((c[0] + c[4]) + (c[2] + c[6])) + ((c[1] + c[5]) + (c[3] + c[7]));
}

// Q8_0 / Q4_0 / Q5_0 on the f16 matrix cores. The reference's integer part
// per block is, for each of the 8 lanes of its accumulator, a sum of 4
// consecutive products P_l (exact: |q| <= 127, |P_l| <= 64516). Here one
// v_mfma_f32_16x16x32_f16 forms P for 4 rows x 16 tokens x 4 of the 8
// groups: A holds the 4 rows' block in group-diagonal form (M index 4r + i
// carries group 2i, or 2i + 1 in the odd product, every other entry zero),
// B the 16 tokens' activations; the values are integers exact in f16 and
// every partial sum is an integer below 2^24, so the f32 result is P itself.
// Lane (q, n) then owns the 8 chains of row q and token n: the f32 fold
// acc_l = fma(f16(d) * y.d, P_l, acc_l) over blocks in order and the avx2
// horizontal sum run on the VALU exactly as in the matvec.
// Wave = SETS sets of 4 rows x TILES tiles of 16 tokens; block = 4 waves
// over BR rows x 64 tokens. The activations arrive as f16 (ActQ8_0::xh,
// written by the batch's quantizer), the weights are converted to f16 when
// staged; both are
// staged in LDS, BS blocks per stage (2 or 4 by the matrix height), two
// stages in LDS and two more in registers in flight.
constexpr int MQ_BS = 2;   // blocks of 32 per stage
constexpr int MQ_XS = 40;  // halves per (block, token) line of the activation tile (32 + pad)

typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f4_t __attribute__((ext_vector_type(4)));

// four unsigned bytes u_i -> the f16 values u_i - bias (exact for u, bias < 1024)
__device__ __forceinline__ void u8x4_to_f16(uint32_t u, float bias, uint32_t &lo, uint32_t &hi) {
    // 0x64 above each byte: the half 1024 + u_i
    const uint32_t l = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t h = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const h2_t off = {(_Float16)(-1024.0f - bias), (_Float16)(-1024.0f - bias)};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, l) + off);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2_t, h) + off);
}

template <int KIND, int SETS, int TILES, int BS = MQ_BS>
__global__ __launch_bounds__(256) void k_mm_q8(MvArgs a, int m) {
    constexpr int WTW = 4 / TILES;      // waves along the tokens
    constexpr int WRW = 4 / WTW;        // waves along the rows
    constexpr int BR = WRW * 4 * SETS;  // weight rows per block
    constexpr int QB = KIND == AOTK_Q8_0 ? 32 : 16;  // quant bytes per block
    constexpr int WPT = KIND == AOTK_Q8_0 ? 2 : 1;   // 16-byte quant loads per (row, block)
    constexpr int WT = BR * BS * WPT;                // weight staging loads per stage
    constexpr int WP = (WT + 255) / 256;             // ... per thread
    constexpr int YP = (64 * BS + 255) / 256;        // activation scales per thread
    static_assert((BS & (BS - 1)) == 0, "stage blocks");
    __shared__ __align__(16) _Float16 sx[2][BS][64][MQ_XS];  // activations
    __shared__ __align__(16) float sxd[2][BS][64];           // their scales
    __shared__ __align__(16) _Float16 sw[2][BR][BS][32];     // weight quants
    __shared__ __align__(16) float swd[2][BR][BS];           // f32(d)
    __shared__ __align__(16) _Float16 szero[8];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = wave / WTW, wt = wave % WTW;
    const int t0 = blockIdx.y * 64;
    const int nb = a.nb;
    const int row0 = blockIdx.x * BR;
    const int mt = min(64, m - t0);
    if (tid < 4) ((uint32_t *)szero)[tid] = 0u;
    // the weight rows / blocks / 16-byte parts this thread stages (pass k: c = tid + 256 k)
    const uint8_t *wq[WP];
    const uint16_t *wd[WP];
    const uint32_t *wh[WP];
#pragma unroll
    for (int k = 0; k < WP; k++) {
        const int c = min(tid + 256 * k, WT - 1);
        const int grow = min(row0 + c / (WPT * BS), a.total_rows - 1);
        int local;
        const int sg = seg_of(a, grow, local);
        wq[k] = seg_sel(sg, a.w[0], a.w[1], a.w[2]) + (size_t)local * nb * QB;
        wd[k] = (const uint16_t *)seg_sel(sg, a.w1[0], a.w1[1], a.w1[2]) + (size_t)local * nb;
        wh[k] = KIND == AOTK_Q5_0 ? (const uint32_t *)seg_sel(sg, a.w2[0], a.w2[1], a.w2[2]) + (size_t)local * nb : nullptr;
    }
    // stage loads (tokens past m and blocks past the end repeat the last:
    // valid memory, never stored)
    struct Ld {
        u32x4_t x[BS], w[WP];
        float xd[YP];
        uint32_t wd[WP], wh[WP];
    };
    Ld L[2];
    auto fetch = [&](Ld &ld, int c0) {
#pragma unroll
        for (int k = 0; k < BS; k++) {  // 64 tokens x BS blocks x 4 parts of 16 bytes
            const int c = tid + 256 * k;
            const int t = min(t0 + c / (4 * BS), m - 1), b = min(c0 + ((c >> 2) & (BS - 1)), nb - 1);
            ld.x[k] = *(const u32x4_t *)(a.xh + (size_t)t * a.cols + (size_t)b * 32 + (c & 3) * 8);
        }
#pragma unroll
        for (int k = 0; k < YP; k++) {
            const int c = tid + 256 * k;  // (token c / BS, block c % BS)
            if (c < 64 * BS) {
                const int t = min(t0 + c / BS, m - 1), b = min(c0 + (c & (BS - 1)), nb - 1);
                ld.xd[k] = a.xd[(size_t)t * nb + b];
            }
        }
#pragma unroll
        for (int k = 0; k < WP; k++) {
            const int c = tid + 256 * k;  // (row c / (WPT BS), block (c / WPT) % BS, part c % WPT)
            if (c < WT) {
                const int part = c % WPT, b = min(c0 + (c / WPT) % BS, nb - 1);
                ld.w[k] = *(const u32x4_t *)(wq[k] + (size_t)b * QB + part * 16);
                if (KIND == AOTK_Q5_0) ld.wh[k] = wh[k][b];
                if (part == 0) ld.wd[k] = wd[k][b];
            }
        }
    };
    auto put = [&](const Ld &ld, int st) {
#pragma unroll
        for (int k = 0; k < BS; k++) {
            const int c = tid + 256 * k;
            *(u32x4_t *)&sx[st][(c >> 2) & (BS - 1)][c / (4 * BS)][(c & 3) * 8] = ld.x[k];
        }
#pragma unroll
        for (int k = 0; k < YP; k++) {
            const int c = tid + 256 * k;
            if (c < 64 * BS) sxd[st][c & (BS - 1)][c / BS] = ld.xd[k];
        }
#pragma unroll
        for (int k = 0; k < WP; k++) {
            const int c = tid + 256 * k;
            if (c >= WT) continue;
            const int part = c % WPT, blk = (c / WPT) % BS, row = c / (WPT * BS);
            uint32_t *dst = (uint32_t *)&sw[st][row][blk][part * 16];
            if (KIND == AOTK_Q8_0) {
                uint32_t h[8];
#pragma unroll
                for (int i = 0; i < 4; i++) u8x4_to_f16(ld.w[k][i] ^ 0x80808080u, 128.0f, h[2 * i], h[2 * i + 1]);
                *(u32x4_t *)dst = u32x4_t{h[0], h[1], h[2], h[3]};
                *(u32x4_t *)(dst + 4) = u32x4_t{h[4], h[5], h[6], h[7]};
            } else {
                // elements 0..15: low nibbles, 16..31: high nibbles (quant.rs:300-443)
                uint32_t h[16];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    uint32_t l4 = ld.w[k][i] & 0x0F0F0F0Fu, h4 = (ld.w[k][i] >> 4) & 0x0F0F0F0Fu;
                    if (KIND == AOTK_Q5_0) {
                        const uint32_t bl = (ld.wh[k] >> (4 * i)) & 0xFu, bh = (ld.wh[k] >> (16 + 4 * i)) & 0xFu;
                        l4 |= ((bl & 1u) | ((bl & 2u) << 7) | ((bl & 4u) << 14) | ((bl & 8u) << 21)) << 4;
                        h4 |= ((bh & 1u) | ((bh & 2u) << 7) | ((bh & 4u) << 14) | ((bh & 8u) << 21)) << 4;
                    }
                    const float bias = KIND == AOTK_Q5_0 ? 16.0f : 8.0f;
                    u8x4_to_f16(l4, bias, h[2 * i], h[2 * i + 1]);
                    u8x4_to_f16(h4, bias, h[8 + 2 * i], h[8 + 2 * i + 1]);
                }
#pragma unroll
                for (int i = 0; i < 4; i++) *(u32x4_t *)(dst + 4 * i) = u32x4_t{h[4 * i], h[4 * i + 1], h[4 * i + 2], h[4 * i + 3]};
            }
            if (part == 0) swd[st][row][blk] = f16_to_f32(ld.wd[k]);
        }
    };
    // lane roles: q = lane / 16 (the output row in a set of 4, and the
    // operands' k-quarter), n = lane % 16 (the token in a tile; as an A row
    // index, row n / 4 of the set with group pair n % 4)
    const int q = lane >> 4, n = lane & 15;
    const bool a_on = (n & 3) == q;  // A[4r + i][k] is nonzero only in k-quarter i
    const int a_row = n >> 2;
    f4_t acc[SETS][TILES][2];  // [row set][token tile][even / odd groups]
#pragma unroll
    for (int s = 0; s < SETS; s++)
#pragma unroll
        for (int t = 0; t < TILES; t++) acc[s][t][0] = acc[s][t][1] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
    fetch(L[0], 0);
    if (BS < nb) fetch(L[1], BS);
    put(L[0], 0);
    __syncthreads();
    // one stage: stage c0 + 2 * BS goes into the register set `fr` just
    // emptied, the stage in `pr` (fetched a round earlier) into the other
    // LDS buffer after the compute (last read in the previous round, before
    // its barrier)
    auto round = [&](int c0, int st, Ld &fr, const Ld &pr) {
        if (c0 + 2 * BS < nb) fetch(fr, c0 + 2 * BS);
        const int nblk = nb - c0 < BS ? nb - c0 : BS;
        for (int j = 0; j < nblk; j++) {
            h8_t bx[TILES];
            float yd[TILES];
#pragma unroll
            for (int t = 0; t < TILES; t++) {
                const int tok = 16 * (wt * TILES + t) + n;
                bx[t] = *(const h8_t *)&sx[st][j][tok][8 * q];
                yd[t] = sxd[st][j][tok];
            }
#pragma unroll
            for (int s = 0; s < SETS; s++) {
                const int r0 = 4 * (wr * SETS + s);  // first row of the set in the block
                const _Float16 *ap = a_on ? &sw[st][r0 + a_row][j][8 * q] : szero;
                const h4_t lo = *(const h4_t *)ap, hi = *(const h4_t *)(ap + 4);
                const _Float16 z = (_Float16)0;
                const h8_t ae = {lo[0], lo[1], lo[2], lo[3], z, z, z, z};
                const h8_t ao = {z, z, z, z, hi[0], hi[1], hi[2], hi[3]};
                const float dw = swd[st][r0 + q][j];
#pragma unroll
                for (int t = 0; t < TILES; t++) {  // (tiles past the batch compute on repeated tokens)
                    const f4_t pe = __builtin_amdgcn_mfma_f32_16x16x32_f16(ae, bx[t], f4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                    const f4_t po = __builtin_amdgcn_mfma_f32_16x16x32_f16(ao, bx[t], f4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                    const float D = dw * yd[t];
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        acc[s][t][0][i] = fmaf(D, pe[i], acc[s][t][0][i]);
                        acc[s][t][1][i] = fmaf(D, po[i], acc[s][t][1][i]);
                    }
                }
            }
        }
        if (c0 + BS < nb) {
            put(pr, st ^ 1);
            __syncthreads();
        }
    };
    for (int c0 = 0; c0 < nb; c0 += 2 * BS) {
        round(c0, 0, L[0], L[1]);
        if (c0 + BS < nb) round(c0 + BS, 1, L[1], L[0]);
    }
    // lane (q, n): row r0 + q of each set, token 16 * tile + n; groups 2i (even) and 2i + 1 (odd)
#pragma unroll
    for (int s = 0; s < SETS; s++) {
        const int grow = row0 + 4 * (wr * SETS + s) + q;
#pragma unroll
        for (int t = 0; t < TILES; t++) {
            const int tt = 16 * (wt * TILES + t) + n;
            const f4_t e = acc[s][t][0], o = acc[s][t][1];
            // ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7))  (simd_avx2.rs:27-34), a_{2i} = e[i], a_{2i+1} = o[i]
            const float v = ((e[0] + e[2]) + (e[1] + e[3])) + ((o[0] + o[2]) + (o[1] + o[3]));
            if (tt < mt && grow < a.total_rows) store_row(a, grow, t0 + tt, v);
        }
    }
}

template <int KIND>
static void launch_mm_q8(const MvArgs &a, int m, hipStream_t s) {
    // (the quants as f16 come with the batch: written by its quantizer)
    // rows per block by the matrix height: enough waves for few rows, more
    // reuse of each staged activation for many
    const unsigned gy = (unsigned)((m + 63) / 64);
    // (sets, tiles, blocks per stage) measured at 64 tokens: 4096 rows
    // (1, 2, 4) against (2, 1, 2) 46 / 59 us at 4096 columns, 126 / 164 us
    // at 12288; 6144 rows (2, 2, 4) 63 against 72 us; 24576 rows (2, 4, 2)
    // 137 against 142 us for 4 blocks per stage
#define Q8L(S, T, B) k_mm_q8<KIND, S, T, B><<<dim3((unsigned)((a.total_rows + 4 * S * T - 1) / (4 * S * T)), gy), 256, 0, s>>>(a, m)
    if (a.total_rows >= 16384) Q8L(2, 4, 2);
    else if (a.total_rows >= 6144) Q8L(2, 2, 4);
    else Q8L(1, 2, 4);
#undef Q8L
}

// F16 / BF16 / F32 rows (4-byte aligned rows): stage = 64 elements x 64
// tokens of f32 input.
template <int KIND>
__global__ __launch_bounds__(256) void k_mm_float(MvArgs a, int m) {
    __shared__ __align__(16) float sx[2][8][64][8];  // [stage][group of 8][token][element]
    constexpr int R = MQ_R;
    constexpr int EB = KIND == AOTK_F32 ? 4 : 2;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t0 = blockIdx.y * 64;
    const int cols = (int)a.cols;
    const int n8 = cols >> 3;
    const int grow0 = (blockIdx.x * 4 + wave) * R;
    const uint8_t *wr[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
        int local;
        const int sg = seg_of(a, grow0 + r < a.total_rows ? grow0 + r : 0, local);
        wr[r] = seg_sel(sg, a.w[0], a.w[1], a.w[2]) + (size_t)local * a.rb;
    }
    // stage loads: 64 tokens x 64 elements, 16 floats per thread (runs of
    // 64 consecutive elements: coalesced, any alignment); elements past the
    // end repeat the last one (never used)
    float lx[16];
    auto fetch = [&](int g0) {
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int j = tid + 256 * k;  // (token j >> 6, element j & 63 of the stage)
            const int t = min(t0 + (j >> 6), m - 1);
            const int e = min(8 * g0 + (j & 63), cols - 1);
            lx[k] = a.xf[(size_t)t * cols + e];
        }
    };
    auto put = [&](int st) {
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int j = tid + 256 * k;
            sx[st][(j & 63) >> 3][j >> 6][j & 7] = lx[k];
        }
    };
    float acc[R][8];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
        for (int l = 0; l < 8; l++) acc[r][l] = 0.0f;
    if (n8 > 0) {
        fetch(0);
        put(0);
    }
    __syncthreads();
    int st = 0;
    for (int g0 = 0; g0 < n8; g0 += 8) {
        const bool more = g0 + 8 < n8;
        if (more) fetch(g0 + 8);
        const int n = n8 - g0 < 8 ? n8 - g0 : 8;
        for (int j = 0; j < n; j++) {
            const int g = g0 + j;
            const float4 x0 = *(const float4 *)&sx[st][j][lane][0], x1 = *(const float4 *)&sx[st][j][lane][4];
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int r = 0; r < R; r++) {
                float wv[8];
                if (KIND == AOTK_F32) {
                    const u32x8_t v = uload<u32x8_t>(wr[r] + (size_t)g * 32);
#pragma unroll
                    for (int l = 0; l < 8; l++) wv[l] = __uint_as_float(v[l]);
                } else {
                    const u32x4_t v = uload<u32x4_t>(wr[r] + (size_t)g * 16);
#pragma unroll
                    for (int l = 0; l < 8; l++) {
                        const uint32_t h = (l & 1) ? v[l >> 1] >> 16 : v[l >> 1] & 0xFFFFu;
                        wv[l] = KIND == AOTK_BF16 ? bf16_to_f32(h) : (float)__builtin_bit_cast(_Float16, (uint16_t)h);
                    }
                }
#pragma unroll
                for (int l = 0; l < 8; l++) acc[r][l] = fmaf(wv[l], xv[l], acc[r][l]);
            }
        }
        if (more) {
            put(st ^ 1);
            __syncthreads();
            st ^= 1;
        }
    }
    const int tok = t0 + lane;
    const int tc = min(tok, m - 1);
#pragma unroll
    for (int r = 0; r < R; r++) {
        float sum = hsum8(acc[r]);
        for (int i = n8 * 8; i < cols; i++) {  // the scalar tail: sum += w * x
            float w;
            if (KIND == AOTK_F32) w = ((const float *)wr[r])[i];
            else {
                const uint32_t h = ((const uint16_t *)wr[r])[i];
                w = KIND == AOTK_BF16 ? bf16_to_f32(h) : (float)__builtin_bit_cast(_Float16, (uint16_t)h);
            }
            const float p = w * a.xf[(size_t)tc * cols + i];
            sum = sum + p;
        }
        if (tok < m && grow0 + r < a.total_rows) store_row(a, grow0 + r, tok, sum);
    }
}

static bool mm_float_fits(const MvArgs &a, int kind) {
    const size_t eb = kind == AOTK_F32 ? 4 : 2;
    if ((a.cols * eb) % 4 != 0) return false;
    for (int i = 0; i < a.nseg; i++)
        if ((uintptr_t)a.w[i] % 4 != 0) return false;
    return true;
}

// ----------------------------------------------------------------- launch

static size_t q8b_lds(const MvArgs &a) { return a.cols + a.cols / 32 * sizeof(float); }

static MvArgs make_args(int n, const DevWeight *const ws[], float *const ys[], const float *const adds[], const void *x_act) {
    MvArgs a = {};
    const DevWeight &w0 = *ws[0];
    a.nseg = n;
    a.total_rows = 0;
    for (int i = 0; i < n; i++) {
        a.w[i] = ws[i]->plane[0];
        a.w1[i] = ws[i]->plane[1];
        a.w2[i] = ws[i]->plane[2];
        a.y[i] = ys[i];
        a.add[i] = adds ? adds[i] : nullptr;
        a.rows[i] = (int)ws[i]->rows;
        a.total_rows += (int)ws[i]->rows;
    }
    a.nb = (int)w0.nb;
    a.rb = row_bytes(w0.kind, w0.cols);
    a.cols = w0.cols;
    int act = activation(w0.kind);
    if (act == ACT_Q8_K) {
        ActQ8K q = *(const ActQ8K *)x_act;
        a.xq = q.qs;
        a.xd = q.d;
        a.xbs = q.bsums;
        a.xt = q.qt;
    } else if (act == ACT_Q8_0) {
        ActQ8_0 q = *(const ActQ8_0 *)x_act;
        a.xq = q.qs;
        a.xd = q.d;
        a.xh = q.xh;
    } else {
        a.xf = (const float *)x_act;
    }
    return a;
}

// Row slots per wave (RL), row groups per wave (G) and blocks of the
// K-quant kernel. One row group per wave at every size: several rounds of
// resident waves measured faster than fewer waves each running G groups with
// the next group's loads in flight (Q4_K 14336x4096 7.8 against 8.8 us with
// three waves per SIMD in one round, the 128256x4096 lm-head 48.4 against
// 49.9 us with two groups per wave).
static bool nb_specialized(int nb) {
    return nb == 8 || nb == 10 || nb == 16 || nb == 22 || nb == 40 || nb == 48 || nb == 56;
}

static void kq_shape(const MvArgs &a, int &RL, int &G, int &blocks) {
    // rows per group: every lane slot of spl * nb lanes that fits
    RL = 64 / (kq_spl(nb_specialized(a.nb) ? a.nb : 0) * a.nb);
    const int groups = (a.total_rows + RL - 1) / RL;
    G = 1;
    blocks = (groups + 3) / 4;
}

template <int KIND>
static void launch_kq(const MvArgs &a, dim3 grid, hipStream_t s) {
    // Q6_K rows of 40..56 super-blocks: two waves per row (the lighter
    // Q4_K / Q5_K terms measured faster on one lane per super-block)
    if (KIND == AOTK_Q6_K && !a.xq_src && (a.nb == 40 || a.nb == 48 || a.nb == 56)) {
        grid.x = (unsigned)((a.total_rows + 1) / 2);
        if (a.nb == 40) k_mv_kqw<KIND, 40><<<grid, 256, 0, s>>>(a);
        else if (a.nb == 48) k_mv_kqw<KIND, 48><<<grid, 256, 0, s>>>(a);
        else k_mv_kqw<KIND, 56><<<grid, 256, 0, s>>>(a);
        return;
    }
    if (a.nb <= 64) {
        int RL, G, blocks;
        kq_shape(a, RL, G, blocks);
        grid.x = (unsigned)blocks;
        // one group per wave: no next-group registers (more waves resident),
        // except for Q6_K rows of one lane per super-block, measured faster
        // with the loads of a second register set in flight
        const bool pf0 = G == 1 && !(KIND == AOTK_Q6_K && kq_spl(a.nb) == 1);
        if (a.xq_src && pf0) {
#define F(NB) k_mv_kq<KIND, 0, NB, true><<<grid, 256, 0, s>>>(a, RL, G)
            AOTK_NB_SWITCH(a.nb, F)
#undef F
        } else if (a.xq_src) {
#define F(NB) k_mv_kq<KIND, 1, NB, true><<<grid, 256, 0, s>>>(a, RL, G)
            AOTK_NB_SWITCH(a.nb, F)
#undef F
        } else if (pf0) {
#define F(NB) k_mv_kq<KIND, 0, NB><<<grid, 256, 0, s>>>(a, RL, G)
            AOTK_NB_SWITCH(a.nb, F)
#undef F
        } else {
#define F(NB) k_mv_kq<KIND, 1, NB><<<grid, 256, 0, s>>>(a, RL, G)
            AOTK_NB_SWITCH(a.nb, F)
#undef F
        }
    } else {
        grid.x = (unsigned)((a.total_rows + 7) / 8);
        k_mv_kquant<KIND, 2><<<grid, 256, 0, s>>>(a);
    }
}

// Persistent k_mm_kx: one round of resident blocks (the occupancy of the
// instance on this device, queried once) walks the 16-row groups.
template <int KIND, int W>
static void launch_mm_kx(const MvArgs &a, int m, hipStream_t s) {
    static int resident = 0;
    if (!resident) {
        int dev = 0, cus = 0, per = 0;
        (void)hipGetDevice(&dev);
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k_mm_kx<KIND, W>, 64 * W, 0);
        resident = std::max(1, cus) * std::max(1, per);
    }
    const int groups = (a.total_rows + 15) / 16;
    k_mm_kx<KIND, W><<<dim3((unsigned)std::min(groups, resident)), 64 * W, 0, s>>>(a, m);
}

static void launch_args(int kind, const MvArgs &a, size_t m, hipStream_t s) {
    dim3 grid;
    grid.y = (unsigned)m;
    if (m >= MM_MIN_TOKENS && m <= MM_TOK && (kind == AOTK_Q4_K || kind == AOTK_Q5_K || kind == AOTK_Q6_K)) {
        // 64 rows per block; the token tiles per block are cut until the
        // grid reaches 512 blocks (small matrices) or one tile is left
        const unsigned rb = (unsigned)((a.total_rows + 63) / 64);
        const int tiles = (int)((m + 15) / 16);
        // few rows (measured: 1024-row v at 64 tokens 2x faster, 4096-row
        // Q6_K down slightly faster, 4096-row Q4_K wo slightly slower):
        // super-blocks split over the waves
        const unsigned cells = rb * (unsigned)tiles;
        // 2048 rows or more with the tiled input: k_mm_kx (measured at 64
        // tokens against the LDS-staged k_mm_kq family: the 4096-row Q4_K
        // wo 16.0 -> 10.4 us, the 28672-row gate/up 73 -> 50 us, the
        // 4096-row Q6_K down 61 -> 41 us; blocks of 4 waves for the tallest
        // Q4_K/Q5_K matrices, of 8 otherwise)
        if (a.total_rows >= 2048 && a.nb <= MMX_MAX_NB && a.xt) {
            const bool tall = a.total_rows >= 16384;
            switch (kind) {
            case AOTK_Q4_K: tall ? launch_mm_kx<AOTK_Q4_K, 4>(a, (int)m, s) : launch_mm_kx<AOTK_Q4_K, 8>(a, (int)m, s); break;
            case AOTK_Q5_K: tall ? launch_mm_kx<AOTK_Q5_K, 4>(a, (int)m, s) : launch_mm_kx<AOTK_Q5_K, 8>(a, (int)m, s); break;
            default: launch_mm_kx<AOTK_Q6_K, 8>(a, (int)m, s); break;
            }
            return;
        }
        if (cells < 128 || (cells <= 256 && a.nb >= 32)) {
            dim3 gk((unsigned)((a.total_rows + 15) / 16), (unsigned)tiles);
            switch (kind) {
            case AOTK_Q4_K: k_mm_ks<AOTK_Q4_K, 1><<<gk, 256, 0, s>>>(a, (int)m); break;
            case AOTK_Q5_K: k_mm_ks<AOTK_Q5_K, 1><<<gk, 256, 0, s>>>(a, (int)m); break;
            default: k_mm_ks<AOTK_Q6_K, 1><<<gk, 256, 0, s>>>(a, (int)m); break;
            }
            return;
        }
        int tt = tiles;
        while (tt > 1 && rb * (unsigned)((tiles + tt - 1) / tt) < 512) tt = (tt + 1) / 2;
        dim3 g(rb, (unsigned)((tiles + tt - 1) / tt));
#define MMK(K)                                                      \
    switch (tt) {                                                   \
    case 1: k_mm_kq<K, 1><<<g, 256, 0, s>>>(a, (int)m); break;      \
    case 2: k_mm_kq<K, 2><<<g, 256, 0, s>>>(a, (int)m); break;      \
    case 3: k_mm_kq<K, 3><<<g, 256, 0, s>>>(a, (int)m); break;      \
    default: k_mm_kq<K, 4><<<g, 256, 0, s>>>(a, (int)m); break;     \
    }
        switch (kind) {
        case AOTK_Q4_K: MMK(AOTK_Q4_K) break;
        case AOTK_Q5_K: MMK(AOTK_Q5_K) break;
        default: MMK(AOTK_Q6_K) break;
        }
#undef MMK
        return;
    }
    if (m >= MM_MIN_TOKENS && (((kind == AOTK_Q8_0 || kind == AOTK_Q4_0 || kind == AOTK_Q5_0) && a.xh) ||
                               ((kind == AOTK_F16 || kind == AOTK_BF16 || kind == AOTK_F32) && mm_float_fits(a, kind)))) {
        dim3 g((unsigned)((a.total_rows + 4 * MQ_R - 1) / (4 * MQ_R)), (unsigned)((m + 63) / 64));
        switch (kind) {
        case AOTK_Q8_0: launch_mm_q8<AOTK_Q8_0>(a, (int)m, s); break;
        case AOTK_Q4_0: launch_mm_q8<AOTK_Q4_0>(a, (int)m, s); break;
        case AOTK_Q5_0: launch_mm_q8<AOTK_Q5_0>(a, (int)m, s); break;
        case AOTK_F16: k_mm_float<AOTK_F16><<<g, 256, 0, s>>>(a, (int)m); break;
        case AOTK_BF16: k_mm_float<AOTK_BF16><<<g, 256, 0, s>>>(a, (int)m); break;
        default: k_mm_float<AOTK_F32><<<g, 256, 0, s>>>(a, (int)m); break;
        }
        return;
    }
    switch (kind) {
    case AOTK_Q4_K:
        launch_kq<AOTK_Q4_K>(a, grid, s);
        break;
    case AOTK_Q5_K:
        launch_kq<AOTK_Q5_K>(a, grid, s);
        break;
    case AOTK_Q6_K:
        launch_kq<AOTK_Q6_K>(a, grid, s);
        break;
    case AOTK_Q8_0:
        if (a.cols <= (size_t)Q8B_MAX_COLS) {
            grid.x = (unsigned)((a.total_rows + 4 * Q8B_R - 1) / (4 * Q8B_R));
            if (a.total_rows >= 65536) k_mv_q8b<AOTK_Q8_0, false, false><<<grid, 256, q8b_lds(a), s>>>(a);
            else k_mv_q8b<AOTK_Q8_0><<<grid, 256, q8b_lds(a), s>>>(a);
        } else {
            grid.x = (unsigned)((a.total_rows + 31) / 32);
            k_mv_q80<AOTK_Q8_0><<<grid, 256, 0, s>>>(a);
        }
        break;
    case AOTK_Q4_0:
        if (a.cols <= (size_t)Q8B_MAX_COLS) {
            grid.x = (unsigned)((a.total_rows + 4 * Q8B_R - 1) / (4 * Q8B_R));
            k_mv_q8b<AOTK_Q4_0><<<grid, 256, q8b_lds(a), s>>>(a);
        } else {
            grid.x = (unsigned)((a.total_rows + 31) / 32);
            k_mv_q80<AOTK_Q4_0><<<grid, 256, 0, s>>>(a);
        }
        break;
    case AOTK_Q5_0:
        if (a.cols <= (size_t)Q8B_MAX_COLS) {
            grid.x = (unsigned)((a.total_rows + 4 * Q8B_R - 1) / (4 * Q8B_R));
            k_mv_q8b<AOTK_Q5_0><<<grid, 256, q8b_lds(a), s>>>(a);
        } else {
            grid.x = (unsigned)((a.total_rows + 31) / 32);
            k_mv_q80<AOTK_Q5_0><<<grid, 256, 0, s>>>(a);
        }
        break;
    case AOTK_F16:
    case AOTK_BF16: {
        grid.x = (unsigned)((a.total_rows + 31) / 32);
        const bool bf = kind == AOTK_BF16;
        if (mv_half_fits(a)) {
            const int n8 = (int)(a.cols >> 3);
            const size_t lds = 8 * sizeof(float) * (size_t)(((n8 + 31) & ~31) + 4);
            // deeper prefetch when few rows leave few waves in flight
            if (a.total_rows < 16384) {
                if (bf) k_mv_half<AOTK_BF16, 8><<<grid, 256, lds, s>>>(a);
                else k_mv_half<AOTK_F16, 8><<<grid, 256, lds, s>>>(a);
            } else {
                if (bf) k_mv_half<AOTK_BF16, 4><<<grid, 256, lds, s>>>(a);
                else k_mv_half<AOTK_F16, 4><<<grid, 256, lds, s>>>(a);
            }
        } else if (bf) {
            k_mv_float<AOTK_BF16><<<grid, 256, 0, s>>>(a);
        } else {
            k_mv_float<AOTK_F16><<<grid, 256, 0, s>>>(a);
        }
        break;
    }
    default:
        grid.x = (unsigned)((a.total_rows + 31) / 32);
        k_mv_float<AOTK_F32><<<grid, 256, 0, s>>>(a);
        break;
    }
}

void launch_matvec(const DevWeight &w, const void *x_act, size_t m, float *y, const float *add, hipStream_t s) {
    const DevWeight *ws[1] = {&w};
    float *ys[1] = {y};
    const float *adds[1] = {add};
    MvArgs a = make_args(1, ws, ys, adds, x_act);
    launch_args(w.kind, a, m, s);
}

void launch_matvec_multi(int n, const DevWeight *const ws[], float *const ys[], const void *x_act, size_t m,
                         hipStream_t s) {
    MvArgs a = make_args(n, ws, ys, nullptr, x_act);
    launch_args(ws[0]->kind, a, m, s);
}

bool launch_matvec_quant(const DevWeight &w, const float *x, float *y, const float *add, hipStream_t s) {
    const int kind = w.kind;
    const DevWeight *ws[1] = {&w};
    float *ys[1] = {y};
    const float *adds[1] = {add};
    if (kind == AOTK_Q8_0 || kind == AOTK_Q4_0 || kind == AOTK_Q5_0) {
        if (w.cols % 256 != 0 || w.cols > (size_t)Q8B_MAX_COLS) return false;
        ActQ8_0 none = {};
        MvArgs a = make_args(1, ws, ys, adds, &none);
        a.xq_src = x;
        const dim3 grid((unsigned)((a.total_rows + 4 * Q8B_R - 1) / (4 * Q8B_R)), 1);
        if (kind == AOTK_Q8_0) k_mv_q8b<AOTK_Q8_0, true><<<grid, 256, q8b_lds(a), s>>>(a);
        else if (kind == AOTK_Q4_0) k_mv_q8b<AOTK_Q4_0, true><<<grid, 256, q8b_lds(a), s>>>(a);
        else k_mv_q8b<AOTK_Q5_0, true><<<grid, 256, q8b_lds(a), s>>>(a);
        return true;
    }
    if ((kind != AOTK_Q4_K && kind != AOTK_Q5_K && kind != AOTK_Q6_K) || w.nb > 64)
        return false;
    ActQ8K none = {};
    MvArgs a = make_args(1, ws, ys, adds, &none);
    a.xq_src = x;
    dim3 grid(1, 1);
    if (kind == AOTK_Q4_K) launch_kq<AOTK_Q4_K>(a, grid, s);
    else if (kind == AOTK_Q5_K) launch_kq<AOTK_Q5_K>(a, grid, s);
    else launch_kq<AOTK_Q6_K>(a, grid, s);
    return true;
}

bool matvec_pair_ok(const DevWeight &a, const DevWeight &b) {
    return ((a.kind == AOTK_Q4_K || a.kind == AOTK_Q5_K) && b.kind == AOTK_Q6_K) && a.cols == b.cols && a.nb <= 64;
}

template <int KA>
static void launch_mm_kx2(const MvArgs &a, const MvArgs &b, int groups, int m, hipStream_t s) {
    static int resident = 0;
    if (!resident) {
        int dev = 0, cus = 0, per = 0;
        (void)hipGetDevice(&dev);
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k_mm_kx2<KA, AOTK_Q6_K, 8>, 512, 0);
        resident = std::max(1, cus) * std::max(1, per);
    }
    k_mm_kx2<KA, AOTK_Q6_K, 8><<<dim3((unsigned)std::min(groups, resident)), 512, 0, s>>>(a, b, m);
}

void launch_matvec_pair(int na, const DevWeight *const wa[], float *const ya[], const DevWeight &wb, float *yb,
                        const void *x_act, size_t m, hipStream_t s) {
    if (m >= MM_MIN_TOKENS) {  // batches: the MFMA matmul per kind
        MvArgs a = make_args(na, wa, ya, nullptr, x_act);
        const DevWeight *wbs[1] = {&wb};
        float *ybs[1] = {yb};
        MvArgs b = make_args(1, wbs, ybs, nullptr, x_act);
        if (m <= MM_TOK && a.xt && a.nb <= MMX_MAX_NB && a.total_rows >= 2048) {
            // both on one persistent launch: b's groups fill the blocks a
            // leaves idle in its last round
            const int groups = (a.total_rows + 15) / 16 + (b.total_rows + 15) / 16;
            if (wa[0]->kind == AOTK_Q4_K) launch_mm_kx2<AOTK_Q4_K>(a, b, groups, (int)m, s);
            else launch_mm_kx2<AOTK_Q5_K>(a, b, groups, (int)m, s);
            return;
        }
        launch_args(wa[0]->kind, a, m, s);
        launch_args(wb.kind, b, m, s);
        return;
    }
    MvArgs a = make_args(na, wa, ya, nullptr, x_act);
    const DevWeight *wbs[1] = {&wb};
    float *ybs[1] = {yb};
    MvArgs b = make_args(1, wbs, ybs, nullptr, x_act);
    int RLa, Ga, na_blk, RLb, Gb, nb_blk;
    kq_shape(a, RLa, Ga, na_blk);
    kq_shape(b, RLb, Gb, nb_blk);
    dim3 grid((unsigned)(na_blk + nb_blk), (unsigned)m);
    if (wa[0]->kind == AOTK_Q4_K) {
#define F(NB) k_mv_kq2<AOTK_Q4_K, AOTK_Q6_K, NB, 0><<<grid, 256, 0, s>>>(a, RLa, Ga, b, RLb, Gb, na_blk)
        AOTK_NB_SWITCH(a.nb, F)
#undef F
    } else {
#define F(NB) k_mv_kq2<AOTK_Q5_K, AOTK_Q6_K, NB, 0><<<grid, 256, 0, s>>>(a, RLa, Ga, b, RLb, Gb, na_blk)
        AOTK_NB_SWITCH(a.nb, F)
#undef F
    }
}

}  // namespace aotk
