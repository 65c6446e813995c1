// sampler.hip - token sampling on the device (crates/aot-kernels/src/sampler.rs):
// repetition penalty, temperature, top-k, top-p and the xorshift64* draw.
//
// Candidates are 64-bit keys: the f32::total_cmp order of the scaled logit in
// the high word, the complement of the token id in the low word, so one
// descending sort orders by logit and, among equal logits, by ascending id.
// Top-k runs in two stages: every block sorts a slice of SAMP_SLICE logits in
// LDS and keeps its best kk; merge blocks then sort up to SAMP_MERGE of those
// at a time and keep the best kk, until one list of kk remains. The final
// block forms exp(c - max), the sequential sums and the walk of
// sampler.rs:75-100 with one thread for the dependent chains.
#include "device.hpp"
#include "internal.hpp"

namespace aotk {

__device__ __forceinline__ uint32_t total_key(float f) {
    const uint32_t b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_value(uint64_t key) {
    const uint32_t u = (uint32_t)(key >> 32);
    return __uint_as_float((u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u);
}
__device__ __forceinline__ uint32_t key_index(uint64_t key) { return ~(uint32_t)key; }

// Descending bitonic sort of N keys in LDS by the whole block.
template <int N>
__device__ void bitonic_desc(uint64_t *a) {
    for (int k = 2; k <= N; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < N; i += blockDim.x) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const uint64_t x = a[i], y = a[ixj];
                    const bool desc = (i & k) == 0;
                    if (desc ? x < y : x > y) {
                        a[i] = y;
                        a[ixj] = x;
                    }
                }
            }
            __syncthreads();
        }
}

// sampler.rs:53-60: every token of win[max(0, count - rln), count) once per
// occurrence (duplicates compound), in order.
__global__ void k_samp_penalty(float *logits, const uint32_t *win, const uint32_t *count, uint32_t rln, float rp) {
    if (threadIdx.x != 0) return;
    const uint32_t c = *count;
    const uint32_t start = c > rln ? c - rln : 0;
    for (uint32_t j = start; j < c; j++) {
        float *l = logits + win[j];
        const float v = *l;
        *l = v > 0.0f ? v / rp : v * rp;
    }
}

// Stage 1: block b sorts the scaled logits of [b * SAMP_SLICE, ...) and
// writes its best kk keys.
__global__ __launch_bounds__(1024) void k_samp_local(const float *logits, int V, float inv_t, int kk, uint64_t *out) {
    __shared__ uint64_t a[SAMP_SLICE];
    const int base = blockIdx.x * SAMP_SLICE;
    for (int i = threadIdx.x; i < SAMP_SLICE; i += blockDim.x) {
        const int t = base + i;
        a[i] = t < V ? ((uint64_t)total_key(logits[t] * inv_t) << 32) | (uint32_t)~(uint32_t)t : 0ull;
    }
    __syncthreads();
    bitonic_desc<SAMP_SLICE>(a);
    for (int i = threadIdx.x; i < kk; i += blockDim.x) out[(size_t)blockIdx.x * kk + i] = a[i];
}

// Stage 2: block b merges lists [b * per, (b + 1) * per) of kk keys each
// (per * kk <= SAMP_MERGE) into its best kk.
__global__ __launch_bounds__(1024) void k_samp_merge(const uint64_t *in, int nlists, int kk, int per, uint64_t *out) {
    __shared__ uint64_t a[SAMP_MERGE];
    const int l0 = blockIdx.x * per;
    const int nl = min(per, nlists - l0);
    for (int i = threadIdx.x; i < SAMP_MERGE; i += blockDim.x)
        a[i] = i < nl * kk ? in[(size_t)l0 * kk + i] : 0ull;
    __syncthreads();
    bitonic_desc<SAMP_MERGE>(a);
    for (int i = threadIdx.x; i < kk; i += blockDim.x) out[(size_t)blockIdx.x * kk + i] = a[i];
}

// xorshift64* (sampler.rs:38-45)
__device__ __forceinline__ float samp_next_f32(uint64_t *rng) {
    uint64_t r = *rng;
    r ^= r >> 12;
    r ^= r << 25;
    r ^= r >> 27;
    *rng = r;
    const uint64_t v = r * 0x2545F4914F6CDD1Dull;
    return (float)(v >> 40) / (float)(1ull << 24);
}

// sampler.rs:75-100 over the k best keys (sorted descending).
__global__ __launch_bounds__(1024) void k_samp_final(const uint64_t *keys, int k, float top_p, uint64_t *rng,
                                                     uint32_t *tok_out, uint32_t *win, uint32_t *count) {
    __shared__ float e[SAMP_KMAX];
    __shared__ float q[SAMP_KMAX];
    __shared__ float bsum;
    const float mx = key_value(keys[0]);
    for (int i = threadIdx.x; i < k; i += blockDim.x) e[i] = aotk_expf(key_value(keys[i]) - mx);
    __syncthreads();
    if (threadIdx.x == 0) {
        float s = 0.0f;
        for (int i = 0; i < k; i++) s += e[i];
        bsum = s;
    }
    __syncthreads();
    const float sum = bsum;
    if (top_p < 1.0f) {
        for (int i = threadIdx.x; i < k; i += blockDim.x) q[i] = e[i] / sum;
        __syncthreads();
    }
    if (threadIdx.x != 0) return;
    int n = k;
    float s = sum;
    if (top_p < 1.0f) {
        float acc = 0.0f;
        for (int i = 0; i < k; i++) {
            acc += q[i];
            if (acc >= top_p) {
                n = i + 1;
                break;
            }
        }
        s = 0.0f;
        for (int i = 0; i < n; i++) s += e[i];
    }
    const float r = samp_next_f32(rng) * s;
    float acc = 0.0f;
    uint32_t tok = key_index(keys[n - 1]);
    for (int i = 0; i < n; i++) {
        acc += e[i];
        if (acc >= r) {
            tok = key_index(keys[i]);
            break;
        }
    }
    *tok_out = tok;
    const uint32_t c = *count;
    win[c] = tok;
    *count = c + 1;
}

// Greedy picks append to the window as well.
__global__ void k_samp_record(const uint32_t *tok, uint32_t *win, uint32_t *count) {
    const uint32_t c = *count;
    win[c] = *tok;
    *count = c + 1;
}

size_t sampler_scratch_bytes(size_t vocab) {
    const size_t blocks = (vocab + SAMP_SLICE - 1) / SAMP_SLICE;
    return 2 * blocks * SAMP_KMAX * sizeof(uint64_t);
}

void launch_sample(const SampleArgs &p, hipStream_t s) {
    if (p.repeat_penalty != 1.0f && p.repeat_last_n > 0)
        k_samp_penalty<<<1, 64, 0, s>>>(p.logits, p.win, p.count, p.repeat_last_n, p.repeat_penalty);
    if (p.temperature <= 0.0f) {  // sampler.rs:61-63
        launch_argmax(p.logits, p.vocab, p.tok_out, p.argmax_ws, s);
        k_samp_record<<<1, 1, 0, s>>>(p.tok_out, p.win, p.count);
        return;
    }
    const int V = (int)p.vocab;
    const int k = p.k;  // 1 <= k <= SAMP_KMAX, k <= V
    const int kk = min(k, SAMP_SLICE);
    int nlists = (V + SAMP_SLICE - 1) / SAMP_SLICE;
    uint64_t *a = p.scratch, *b = p.scratch + (size_t)nlists * SAMP_KMAX;
    k_samp_local<<<nlists, 1024, 0, s>>>(p.logits, V, 1.0f / p.temperature, kk, a);
    int kp = 1;
    while (kp < kk) kp <<= 1;
    const int per = max(2, SAMP_MERGE / kp);
    while (nlists > 1) {
        const int nb = (nlists + per - 1) / per;
        k_samp_merge<<<nb, 1024, 0, s>>>(a, nlists, kk, per, b);
        nlists = nb;
        uint64_t *t = a;
        a = b;
        b = t;
    }
    k_samp_final<<<1, 1024, 0, s>>>(a, k, p.top_p, p.rng, p.tok_out, p.win, p.count);
}

}  // namespace aotk
