// runtime.hip - the C ABI of libaotk.so (include/aotk.h): device/stream
// management, weights resident in HBM, the per-kernel entry points, and the
// model runtime that replays the generated forward()/forward_batch()
// operator sequence (crates/aot-codegen/src/emit.rs:167-333, :466-516) on
// the GPU. Single stream, no host synchronisation inside a step.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>
#include <stdlib.h>

#include "internal.hpp"

using namespace aotk;

// ------------------------------------------------------------------ errors
// Thread-local last error like capi.rs:129-141.
static thread_local std::string g_err;

static int fail(const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return -1;
}

#define HIPC(call)                                                                        \
    do {                                                                                  \
        hipError_t e_ = (call);                                                           \
        if (e_ != hipSuccess) return fail("%s: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__, __LINE__); \
    } while (0)

#define HIPP(call)                                                                        \
    do {                                                                                  \
        hipError_t e_ = (call);                                                           \
        if (e_ != hipSuccess) {                                                           \
            fail("%s: %s (%s:%d)", #call, hipGetErrorString(e_), __FILE__, __LINE__);    \
            return nullptr;                                                               \
        }                                                                                 \
    } while (0)

static int g_device = -1;
static hipStream_t g_stream = nullptr;
static bool g_decode_graphs = true;  // set by aotk_init

// Library scratch for the per-kernel entry points (grown on demand).
static void *g_scratch = nullptr;
static size_t g_scratch_bytes = 0;

// Staging memory of aotk_matmul_noalloc: a fixed device array (one copy per
// GPU, held until the process ends) instead of the growable scratch above.
// Host code never passes `scratch` itself (its host-side name is not a
// device address): aotk_init looks its address up per device.
static constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(4) << 20;
static constexpr int NOALLOC_MAX_DEVICES = 64;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];
static void *g_noalloc_scratch[NOALLOC_MAX_DEVICES] = {};

static int ensure_init() {
    if (g_stream) return 0;
    return aotk_init(0);
}

static void *lib_scratch(size_t bytes) {
    if (bytes <= g_scratch_bytes) return g_scratch;
    if (g_scratch) (void)hipFree(g_scratch);
    g_scratch = nullptr;
    g_scratch_bytes = 0;
    size_t want = align_up(bytes, 1 << 20);
    if (hipMalloc(&g_scratch, want) != hipSuccess) {
        fail("hipMalloc of %zu scratch bytes failed", want);
        return nullptr;
    }
    g_scratch_bytes = want;
    return g_scratch;
}

extern "C" {

const char *aotk_last_error(void) { return g_err.c_str(); }

int aotk_init(int device) {
    if (g_stream) {
        if (device != g_device) return fail("aotk_init: already initialised on device %d", g_device);
        return 0;
    }
    int n = 0;
    HIPC(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return fail("aotk_init: device %d out of range (%d devices)", device, n);
    if (device >= NOALLOC_MAX_DEVICES) return fail("aotk_init: device %d beyond the supported %d", device, NOALLOC_MAX_DEVICES);
    HIPC(hipSetDevice(device));
    HIPC(hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking));
    g_device = device;
    // the one run-time option: AOTK_NO_GRAPH=1 replays decode loops as plain
    // stream launches (for kernel traces that list every launch)
    const char *ng = getenv("AOTK_NO_GRAPH");
    g_decode_graphs = !(ng && ng[0] && ng[0] != '0');
    void *na = nullptr;
    hipError_t e = hipGetSymbolAddress(&na, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !na) {
        // leave the library uninitialised so that a later call retries
        (void)hipStreamDestroy(g_stream);
        g_stream = nullptr;
        return fail("aotk_init: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    }
    g_noalloc_scratch[device] = na;
    return 0;
}

void *aotk_stream(void) { return (void *)g_stream; }

void *aotk_dev_alloc(size_t bytes) {
    if (ensure_init()) return nullptr;
    void *p = nullptr;
    HIPP(hipMalloc(&p, bytes ? bytes : 1));
    return p;
}

int aotk_dev_free(void *p) {
    if (!p) return 0;
    HIPC(hipFree(p));
    return 0;
}

int aotk_h2d(void *dst, const void *src, size_t bytes) {
    if (ensure_init()) return -1;
    HIPC(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream));
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

int aotk_d2h(void *dst, const void *src, size_t bytes) {
    if (ensure_init()) return -1;
    HIPC(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream));
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

int aotk_d2d(void *dst, const void *src, size_t bytes) {
    if (ensure_init()) return -1;
    HIPC(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_stream));
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

int aotk_memset(void *dst, int value, size_t bytes) {
    if (ensure_init()) return -1;
    HIPC(hipMemsetAsync(dst, value, bytes, g_stream));
    return 0;
}

int aotk_sync(void) {
    if (ensure_init()) return -1;
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

size_t aotk_row_bytes(int kind, size_t cols) { return valid_kind(kind) ? row_bytes(kind, cols) : 0; }

}  // extern "C"

// ------------------------------------------------------------------ weights

struct aotk_weight {
    DevWeight dw;
};

static int check_shape(int kind, size_t rows, size_t cols) {
    if (!valid_kind(kind)) return fail("unknown weight kind %d", kind);
    if (rows == 0 || cols == 0) return fail("empty matrix %zux%zu", rows, cols);
    if (cols % block_size(kind) != 0) return fail("cols %zu is not a multiple of the block size %zu", cols, block_size(kind));
    return 0;
}

static aotk_weight *weight_from_raw_dev(int kind, const void *raw_dev, size_t rows, size_t cols) {
    aotk_weight *w = new aotk_weight();
    w->dw.kind = kind;
    w->dw.rows = rows;
    w->dw.cols = cols;
    uint8_t *base = nullptr;
    if (hipMalloc(&base, weight_dev_bytes(kind, rows, cols)) != hipSuccess) {
        delete w;
        fail("hipMalloc for a %zux%zu weight failed", rows, cols);
        return nullptr;
    }
    weight_set_planes(w->dw, base);
    launch_repack(w->dw, (const uint8_t *)raw_dev, g_stream);
    return w;
}

extern "C" {

aotk_weight *aotk_weight_from_dev(int kind, const void *bytes_dev, size_t rows, size_t cols) {
    if (ensure_init() || check_shape(kind, rows, cols)) return nullptr;
    aotk_weight *w = weight_from_raw_dev(kind, bytes_dev, rows, cols);
    if (w && hipStreamSynchronize(g_stream) != hipSuccess) {
        fail("repack failed");
        return nullptr;
    }
    return w;
}

aotk_weight *aotk_weight_upload(int kind, const void *bytes_host, size_t rows, size_t cols) {
    if (ensure_init() || check_shape(kind, rows, cols)) return nullptr;
    size_t n = rows * row_bytes(kind, cols);
    void *staging = nullptr;
    HIPP(hipMalloc(&staging, n));
    if (hipMemcpyAsync(staging, bytes_host, n, hipMemcpyHostToDevice, g_stream) != hipSuccess) {
        (void)hipFree(staging);
        fail("upload failed");
        return nullptr;
    }
    aotk_weight *w = weight_from_raw_dev(kind, staging, rows, cols);
    (void)hipStreamSynchronize(g_stream);
    (void)hipFree(staging);
    return w;
}

int aotk_weight_free(aotk_weight *w) {
    if (!w) return 0;
    (void)hipStreamSynchronize(g_stream);
    HIPC(hipFree(w->dw.base));
    delete w;
    return 0;
}

int aotk_dequant_rows(const aotk_weight *w, size_t row0, size_t n_rows, float *out_dev) {
    if (!w) return fail("null weight");
    if (row0 + n_rows > w->dw.rows) return fail("rows [%zu, %zu) out of range (%zu rows)", row0, row0 + n_rows, w->dw.rows);
    launch_dequant(w->dw, row0, n_rows, out_dev, g_stream);
    HIPC(hipGetLastError());
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

int aotk_quantize_rows(int kind, const float *x_dev, size_t rows, size_t cols, void *out_dev) {
    if (ensure_init() || check_shape(kind, rows, cols)) return -1;
    launch_encode(kind, x_dev, rows, cols, (uint8_t *)out_dev, g_stream);
    HIPC(hipGetLastError());
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

int aotk_quantize_q8_0(const float *x_dev, size_t n, aotk_block_q8_0 *out_dev) {
    if (ensure_init()) return -1;
    if (n % 32) return fail("quantize_q8_0: n = %zu is not a multiple of 32", n);
    void *s = lib_scratch(act_q8_0_bytes(n, 1));
    if (!s) return -1;
    ActQ8_0 a = act_q8_0_view(s, n, 1);
    launch_quant_q8_0(x_dev, n, 1, a, g_stream);
    launch_q8_0_to_ref(a, n, out_dev, g_stream);
    HIPC(hipGetLastError());
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

int aotk_quantize_q8_k(const float *x_dev, size_t n, aotk_block_q8_k *out_dev) {
    if (ensure_init()) return -1;
    if (n % 256) return fail("quantize_q8_k: n = %zu is not a multiple of 256", n);
    void *s = lib_scratch(act_q8k_bytes(n, 1));
    if (!s) return -1;
    ActQ8K a = act_q8k_view(s, n, 1);
    launch_quant_q8k(x_dev, n, 1, a, g_stream);
    launch_q8k_to_ref(a, n, out_dev, g_stream);
    HIPC(hipGetLastError());
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

}  // extern "C"

// Convert m reference-layout activation vectors into the plane layout;
// returns the view to pass to launch_matvec. The staging memory is the
// library scratch, or `fixed` (fixed_cap bytes) when that is given.
static int stage_act(const DevWeight &w, const void *x_dev, size_t m, ActQ8K &qk, ActQ8_0 &q0, const void *&act,
                     void *fixed = nullptr, size_t fixed_cap = 0) {
    int a = activation(w.kind);
    if (a == ACT_Q8_K || a == ACT_Q8_0) {
        const size_t need = a == ACT_Q8_K ? act_q8k_bytes(w.cols, m) : act_q8_0_bytes(w.cols, m);
        void *s;
        if (fixed) {
            if (need > fixed_cap)
                return fail("matmul_noalloc: %zu inputs of %zu columns need %zu staging bytes, above the fixed %zu", m,
                            w.cols, need, fixed_cap);
            s = fixed;
        } else {
            s = lib_scratch(need);
            if (!s) return -1;
        }
        if (a == ACT_Q8_K) {
            qk = act_q8k_view(s, w.cols, m);
            launch_ref_to_q8k((const aotk_block_q8_k *)x_dev, w.cols, m, qk, g_stream);
            act = &qk;
        } else {
            q0 = act_q8_0_view(s, w.cols, m);
            launch_ref_to_q8_0((const aotk_block_q8_0 *)x_dev, w.cols, m, q0, g_stream);
            act = &q0;
        }
    } else {
        act = x_dev;
    }
    return 0;
}

extern "C" {

int aotk_matvec(const aotk_weight *w, const void *x_dev, float *out_dev) { return aotk_matmul(w, x_dev, 1, out_dev); }

int aotk_matmul(const aotk_weight *w, const void *xs_dev, size_t m, float *out_dev) {
    if (!w) return fail("null weight");
    if (m == 0) return 0;
    ActQ8K qk;
    ActQ8_0 q0;
    const void *act;
    if (stage_act(w->dw, xs_dev, m, qk, q0, act)) return -1;
    launch_matvec(w->dw, act, m, out_dev, nullptr, g_stream);
    HIPC(hipGetLastError());
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

// The fused multi-matrix products: one launch over the concatenated rows of
// matrices of one kind and width sharing one input.
static int multi_product(int n, const aotk_weight *const *ws, const void *xs_dev, size_t m, float *const *outs,
                         const char *what, bool same_rows) {
    for (int i = 0; i < n; i++)
        if (!ws[i] || !outs[i]) return fail("%s: null weight or output", what);
    const DevWeight &w0 = ws[0]->dw;
    for (int i = 1; i < n; i++) {
        const DevWeight &wi = ws[i]->dw;
        if (wi.kind != w0.kind || wi.cols != w0.cols || (same_rows && wi.rows != w0.rows))
            return fail("%s: the matrices differ in kind or shape", what);
    }
    if (m == 0) return 0;
    ActQ8K qk;
    ActQ8_0 q0;
    const void *act;
    if (stage_act(w0, xs_dev, m, qk, q0, act)) return -1;
    const DevWeight *dws[3];
    float *ys[3];
    for (int i = 0; i < n; i++) {
        dws[i] = &ws[i]->dw;
        ys[i] = outs[i];
    }
    launch_matvec_multi(n, dws, ys, act, m, g_stream);
    HIPC(hipGetLastError());
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

int aotk_matvec3(const aotk_weight *const ws[3], const void *x_dev, float *const outs[3]) {
    return multi_product(3, ws, x_dev, 1, outs, "matvec3", false);
}

int aotk_matvec2(const aotk_weight *w_a, const aotk_weight *w_b, const void *x_dev, float *out_a, float *out_b) {
    const aotk_weight *ws[2] = {w_a, w_b};
    float *outs[2] = {out_a, out_b};
    return multi_product(2, ws, x_dev, 1, outs, "matvec2", true);
}

int aotk_matmul2(const aotk_weight *w_a, const aotk_weight *w_b, const void *xs_dev, size_t m, float *out_a,
                 float *out_b) {
    const aotk_weight *ws[2] = {w_a, w_b};
    float *outs[2] = {out_a, out_b};
    return multi_product(2, ws, xs_dev, m, outs, "matmul2", true);
}

int aotk_matmul_noalloc(const aotk_weight *w, const void *xs_dev, size_t m, float *out_dev) {
    if (!w) return fail("null weight");
    if (ensure_init()) return -1;
    if (m == 0) return 0;
    ActQ8K qk;
    ActQ8_0 q0;
    const void *act;
    if (stage_act(w->dw, xs_dev, m, qk, q0, act, g_noalloc_scratch[g_device], NOALLOC_SCRATCH_BYTES)) return -1;
    launch_matvec(w->dw, act, m, out_dev, nullptr, g_stream);
    HIPC(hipGetLastError());
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

int aotk_matvec_f32(const aotk_weight *w, const float *x_dev, float *out_dev) {
    if (!w) return fail("null weight");
    const DevWeight &dw = w->dw;
    // where the kind and width allow, one launch: the matvec quantizes the
    // input itself (the same quants as the separate quantizer below)
    if (launch_matvec_quant(dw, x_dev, out_dev, nullptr, g_stream)) {
        HIPC(hipGetLastError());
        HIPC(hipStreamSynchronize(g_stream));
        return 0;
    }
    int a = activation(dw.kind);
    const void *act = x_dev;
    ActQ8K qk;
    ActQ8_0 q0;
    if (a == ACT_Q8_K) {
        void *s = lib_scratch(act_q8k_bytes(dw.cols, 1));
        if (!s) return -1;
        qk = act_q8k_view(s, dw.cols, 1);
        launch_quant_q8k(x_dev, dw.cols, 1, qk, g_stream);
        act = &qk;
    } else if (a == ACT_Q8_0) {
        void *s = lib_scratch(act_q8_0_bytes(dw.cols, 1));
        if (!s) return -1;
        q0 = act_q8_0_view(s, dw.cols, 1);
        launch_quant_q8_0(x_dev, dw.cols, 1, q0, g_stream);
        act = &q0;
    }
    launch_matvec(dw, act, 1, out_dev, nullptr, g_stream);
    HIPC(hipGetLastError());
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

static int finish_op() {
    HIPC(hipGetLastError());
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

int aotk_rmsnorm(float *out_dev, const float *x_dev, const float *w_dev, size_t n, size_t m, float eps) {
    if (ensure_init()) return -1;
    if (n % 256 || n > 8192) return fail("rmsnorm: n = %zu must be a multiple of 256 and at most 8192", n);
    RmsOut o = {};
    o.f32 = out_dev;
    launch_rmsnorm_quant(x_dev, w_dev, n, m, eps, o, g_stream);
    return finish_op();
}

int aotk_rmsnorm_heads(float *x_dev, const float *w_dev, size_t n_heads, size_t head_dim, float eps) {
    if (ensure_init()) return -1;
    if (head_dim > 256) return fail("rmsnorm_heads: head_dim %zu > 256", head_dim);
    launch_rmsnorm_heads(x_dev, w_dev, n_heads, head_dim, eps, g_stream);
    return finish_op();
}

int aotk_rope(float *x_dev, size_t m, size_t n_heads, size_t head_dim, size_t rot_dim, const float *cs_dev, int neox) {
    if (ensure_init()) return -1;
    if (head_dim > 256 || rot_dim > head_dim || rot_dim % 2) return fail("rope: bad head_dim %zu / rot_dim %zu", head_dim, rot_dim);
    launch_rope(x_dev, m, n_heads, head_dim, rot_dim, cs_dev, neox, g_stream);
    return finish_op();
}

int aotk_softmax(float *x_dev, size_t n) {
    if (ensure_init()) return -1;
    launch_softmax(x_dev, n, g_stream);
    return finish_op();
}

int aotk_silu_mul(float *h_dev, const float *up_dev, size_t n) {
    if (ensure_init()) return -1;
    launch_silu_mul(h_dev, up_dev, n, 0, g_stream);
    return finish_op();
}

int aotk_gelu_mul(float *h_dev, const float *up_dev, size_t n) {
    if (ensure_init()) return -1;
    launch_silu_mul(h_dev, up_dev, n, 1, g_stream);
    return finish_op();
}

int aotk_add(float *x_dev, const float *y_dev, size_t n) {
    if (ensure_init()) return -1;
    launch_add(x_dev, y_dev, n, g_stream);
    return finish_op();
}

int aotk_attention(float *out_dev, const float *q_dev, const float *k_cache_dev, const float *v_cache_dev, size_t n_head,
                   size_t n_kv_head, size_t head_dim, size_t ctx, size_t layer, size_t pos0, size_t m, size_t window) {
    if (ensure_init()) return -1;
    if (head_dim != 64 && head_dim != 128 && head_dim != 256) return fail("attention: head_dim %zu unsupported", head_dim);
    if (n_kv_head == 0 || n_head % n_kv_head || n_head / n_kv_head > 8) return fail("attention: bad head counts");
    if (pos0 + m > ctx) return fail("attention: positions exceed the context");
    if (ctx > 16384) return fail("attention: context %zu exceeds 16384 positions", ctx);
    size_t kv = n_kv_head * head_dim;
    size_t bytes = attention_scratch_bytes(n_head, head_dim, ctx, m);
    void *s = lib_scratch(bytes);
    if (!s) return -1;
    launch_attention(out_dev, q_dev, k_cache_dev + layer * ctx * kv, v_cache_dev + layer * ctx * kv, n_head, n_kv_head,
                     head_dim, ctx, pos0, m, window, nullptr, (float *)s, bytes, g_stream);
    return finish_op();
}

int aotk_argmax(const float *x_dev, size_t n, uint32_t *out_host) {
    if (ensure_init()) return -1;
    uint8_t *s = (uint8_t *)lib_scratch(4096);
    if (!s) return -1;
    launch_argmax(x_dev, n, (uint32_t *)(s + 2048), (float *)s, g_stream);
    HIPC(hipGetLastError());
    HIPC(hipMemcpyAsync(out_host, s + 2048, 4, hipMemcpyDeviceToHost, g_stream));
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

}  // extern "C"

// -------------------------------------------------------------------- model

struct LayerDev {
    DevWeight wq, wk, wv, wo, gate, up, down;
    const float *attn_norm, *ffn_norm, *bq, *bk, *bv, *q_norm, *k_norm, *attn_post_norm, *ffn_post_norm;
    int local_attn;
};

struct aotk_model {
    aotk_model_spec spec;
    std::vector<aotk_layer> layers;
    size_t blob_len;
    uint8_t *arena;
    size_t arena_bytes;
    DevWeight embd, output;
    const float *output_norm;
    std::vector<float> rope_freqs;  // host copy (empty: none)
    std::vector<LayerDev> dev;
    uint64_t weight_bytes;
};

static const char *kind_ok_matrix(const aotk_tensor &t) {
    if (!valid_kind(t.kind)) return "invalid kind";
    if (t.cols % block_size(t.kind)) return "cols not a multiple of the block size";
    if (t.len != t.rows * row_bytes(t.kind, t.cols)) return "len != rows * row_bytes";
    return nullptr;
}

static int validate_spec(const aotk_model_spec *s, size_t blob_len) {
    const aotk_dims &d = s->dims;
    if (d.n_layer == 0 || !s->layers) return fail("spec: no layers");
    if (d.n_kv_head == 0 || d.n_head % d.n_kv_head) return fail("spec: n_head %llu not a multiple of n_kv_head %llu",
                                                                 (unsigned long long)d.n_head, (unsigned long long)d.n_kv_head);
    if (d.n_head / d.n_kv_head > 8) return fail("spec: gqa > 8 unsupported");
    if (d.head_dim != 64 && d.head_dim != 128 && d.head_dim != 256) return fail("spec: head_dim %llu unsupported", (unsigned long long)d.head_dim);
    if (d.head_dim == 256 && d.n_head / d.n_kv_head > 4) return fail("spec: head_dim 256 supports at most 4 query heads per kv head");
    if (d.rot_dim > d.head_dim || d.rot_dim % 2) return fail("spec: bad rot_dim");
    size_t qd = d.n_head * d.head_dim;
    if (d.dim % 256 || d.hidden % 256 || qd % 256 || d.dim > 8192)
        return fail("spec: dim, hidden and q_dim must be multiples of 256 (dim <= 8192)");
    auto chk = [&](const aotk_tensor &t, size_t rows, size_t cols, const char *name, bool vec) -> int {
        if (vec) {
            if (t.kind != AOTK_F32) return fail("spec: %s must be f32", name);
            if (t.rows * t.cols != cols) return fail("spec: %s has %llu elements, expected %zu", name, (unsigned long long)(t.rows * t.cols), cols);
        } else {
            const char *e = kind_ok_matrix(t);
            if (e) return fail("spec: %s: %s", name, e);
            if (t.rows != rows || t.cols != cols) return fail("spec: %s is %llux%llu, expected %zux%zu", name, (unsigned long long)t.rows,
                                                              (unsigned long long)t.cols, rows, cols);
        }
        if (t.off + (vec ? cols * 4 : t.len) > blob_len) return fail("spec: %s lies outside the blob", name);
        if (vec && t.off % 4) return fail("spec: %s is not 4-byte aligned", name);
        return 0;
    };
    size_t kv = d.n_kv_head * d.head_dim;
    if (chk(s->token_embd, d.vocab, d.dim, "token_embd", false)) return -1;
    if (chk(s->output_norm, 1, d.dim, "output_norm", true)) return -1;
    if (s->output.kind != AOTK_KIND_NONE && chk(s->output, d.vocab, d.dim, "output", false)) return -1;
    for (size_t l = 0; l < d.n_layer; l++) {
        const aotk_layer &L = s->layers[l];
        if (chk(L.attn_norm, 1, d.dim, "attn_norm", true) || chk(L.wq, qd, d.dim, "wq", false) || chk(L.wk, kv, d.dim, "wk", false) ||
            chk(L.wv, kv, d.dim, "wv", false) || chk(L.wo, d.dim, qd, "wo", false) || chk(L.ffn_norm, 1, d.dim, "ffn_norm", true) ||
            chk(L.gate, d.hidden, d.dim, "gate", false) || chk(L.up, d.hidden, d.dim, "up", false) || chk(L.down, d.dim, d.hidden, "down", false))
            return -1;
        if (s->flags.qkv_bias && (chk(L.bq, 1, qd, "bq", true) || chk(L.bk, 1, kv, "bk", true) || chk(L.bv, 1, kv, "bv", true))) return -1;
        if (s->flags.qk_norm && (chk(L.q_norm, 1, d.head_dim, "q_norm", true) || chk(L.k_norm, 1, d.head_dim, "k_norm", true))) return -1;
        if (s->flags.post_norms && (chk(L.attn_post_norm, 1, d.dim, "attn_post_norm", true) || chk(L.ffn_post_norm, 1, d.dim, "ffn_post_norm", true)))
            return -1;
    }
    return 0;
}

// Visit every tensor slot of the spec: f(tensor, index, is_matrix, is_norm).
// Tensor index matches the synthetic generator: token_embd 0, output_norm 1,
// output 2, layer l slot s -> 3 + 16*l + s (aotk_layer field order).
template <typename F>
static int for_each_tensor(const aotk_model_spec *s, F f) {
    if (f(s->token_embd, 0u, true, false)) return -1;
    if (f(s->output_norm, 1u, false, true)) return -1;
    if (s->output.kind != AOTK_KIND_NONE && f(s->output, 2u, true, false)) return -1;
    for (size_t l = 0; l < s->dims.n_layer; l++) {
        const aotk_layer &L = s->layers[l];
        const aotk_tensor *slots[16] = {&L.attn_norm, &L.wq, &L.wk, &L.wv, &L.wo, &L.ffn_norm, &L.gate, &L.up, &L.down,
                                        &L.bq, &L.bk, &L.bv, &L.q_norm, &L.k_norm, &L.attn_post_norm, &L.ffn_post_norm};
        static const bool matrix[16] = {false, true, true, true, true, false, true, true, true, false, false, false, false, false, false, false};
        static const bool norm[16] = {true, false, false, false, false, true, false, false, false, false, false, false, true, true, true, true};
        for (int k = 0; k < 16; k++)
            if (slots[k]->kind != AOTK_KIND_NONE && f(*slots[k], (uint32_t)(3 + 16 * l + k), matrix[k], norm[k])) return -1;
    }
    return 0;
}

// Arena layout: every tensor gets weight_dev_bytes (matrices) or its f32 bytes
// (vectors), 256-byte aligned, in spec order. Returns the device address for
// tensor offset `off`.
struct ArenaMap {
    std::vector<std::pair<uint64_t, size_t>> at;  // (blob off, arena off)
    size_t find(uint64_t off) const {
        for (auto &p : at)
            if (p.first == off) return p.second;
        return (size_t)-1;
    }
};

static aotk_model *model_alloc(const aotk_model_spec *spec, size_t blob_len, ArenaMap &map) {
    aotk_model *m = new aotk_model();
    m->spec = *spec;
    m->layers.assign(spec->layers, spec->layers + spec->dims.n_layer);
    m->spec.layers = m->layers.data();
    m->blob_len = blob_len;
    size_t total = 0;
    for_each_tensor(&m->spec, [&](const aotk_tensor &t, uint32_t, bool matrix, bool) {
        if (map.find(t.off) != (size_t)-1) return 0;
        size_t b = matrix ? weight_dev_bytes(t.kind, t.rows, t.cols) : align_up(t.rows * t.cols * 4, 256);
        map.at.push_back({t.off, total});
        total += align_up(b, 256);
        return 0;
    });
    m->arena_bytes = total;
    if (hipMalloc(&m->arena, total) != hipSuccess) {
        fail("hipMalloc of %zu bytes for the weights failed", total);
        delete m;
        return nullptr;
    }
    return m;
}

static DevWeight dev_weight(aotk_model *m, const ArenaMap &map, const aotk_tensor &t) {
    DevWeight w = {};
    w.kind = t.kind;
    w.rows = t.rows;
    w.cols = t.cols;
    weight_set_planes(w, m->arena + map.find(t.off));
    return w;
}

static void model_bind(aotk_model *m, const ArenaMap &map) {
    const aotk_model_spec &s = m->spec;
    m->embd = dev_weight(m, map, s.token_embd);
    m->output = s.output.kind != AOTK_KIND_NONE ? dev_weight(m, map, s.output) : m->embd;
    m->output_norm = (const float *)(m->arena + map.find(s.output_norm.off));
    m->dev.resize(s.dims.n_layer);
    uint64_t wb = 0;
    auto vec = [&](const aotk_tensor &t) -> const float * {
        return t.kind == AOTK_KIND_NONE ? nullptr : (const float *)(m->arena + map.find(t.off));
    };
    for (size_t l = 0; l < s.dims.n_layer; l++) {
        const aotk_layer &L = s.layers[l];
        LayerDev &D = m->dev[l];
        D.wq = dev_weight(m, map, L.wq);
        D.wk = dev_weight(m, map, L.wk);
        D.wv = dev_weight(m, map, L.wv);
        D.wo = dev_weight(m, map, L.wo);
        D.gate = dev_weight(m, map, L.gate);
        D.up = dev_weight(m, map, L.up);
        D.down = dev_weight(m, map, L.down);
        D.attn_norm = vec(L.attn_norm);
        D.ffn_norm = vec(L.ffn_norm);
        D.bq = s.flags.qkv_bias ? vec(L.bq) : nullptr;
        D.bk = s.flags.qkv_bias ? vec(L.bk) : nullptr;
        D.bv = s.flags.qkv_bias ? vec(L.bv) : nullptr;
        D.q_norm = s.flags.qk_norm ? vec(L.q_norm) : nullptr;
        D.k_norm = s.flags.qk_norm ? vec(L.k_norm) : nullptr;
        D.attn_post_norm = s.flags.post_norms ? vec(L.attn_post_norm) : nullptr;
        D.ffn_post_norm = s.flags.post_norms ? vec(L.ffn_post_norm) : nullptr;
        D.local_attn = L.local_attn;
        for (const aotk_tensor *t : {&L.wq, &L.wk, &L.wv, &L.wo, &L.gate, &L.up, &L.down}) wb += t->len;
    }
    const aotk_tensor &ot = s.output.kind != AOTK_KIND_NONE ? s.output : s.token_embd;
    wb += ot.len + row_bytes(s.token_embd.kind, s.token_embd.cols);
    m->weight_bytes = wb;
}

extern "C" {

aotk_model *aotk_model_load(const aotk_model_spec *spec, const void *blob_host, size_t blob_len) {
    if (ensure_init()) return nullptr;
    if (!spec || !blob_host) {
        fail("aotk_model_load: null argument");
        return nullptr;
    }
    if (validate_spec(spec, blob_len)) return nullptr;
    ArenaMap map;
    aotk_model *m = model_alloc(spec, blob_len, map);
    if (!m) return nullptr;
    // Tensor by tensor: each matrix is uploaded into one staging buffer sized
    // to the largest matrix (not the whole blob, so that loading needs the
    // model's HBM plus one tensor) and repacked from there; vectors go
    // straight to their place. The stream orders each upload after the
    // previous repack.
    size_t max_len = 0;
    for_each_tensor(spec, [&](const aotk_tensor &t, uint32_t, bool matrix, bool) {
        if (matrix && t.len > max_len) max_len = t.len;
        return 0;
    });
    uint8_t *staging = nullptr;
    if (hipMalloc(&staging, max_len ? max_len : 1) != hipSuccess) {
        fail("hipMalloc of the %zu-byte upload buffer failed", max_len);
        (void)hipFree(m->arena);
        delete m;
        return nullptr;
    }
    const uint8_t *src = (const uint8_t *)blob_host;
    int rc = for_each_tensor(&m->spec, [&](const aotk_tensor &t, uint32_t, bool matrix, bool) {
        uint8_t *dst = m->arena + map.find(t.off);
        if (matrix) {
            if (hipMemcpyAsync(staging, src + t.off, t.len, hipMemcpyHostToDevice, g_stream) != hipSuccess)
                return fail("uploading a %zu-byte tensor failed", (size_t)t.len);
            DevWeight w = dev_weight(m, map, t);
            launch_repack(w, staging, g_stream);
        } else if (hipMemcpyAsync(dst, src + t.off, t.rows * t.cols * 4, hipMemcpyHostToDevice, g_stream) != hipSuccess) {
            return fail("uploading a %zu-value vector failed", (size_t)(t.rows * t.cols));
        }
        return 0;
    });
    hipError_t e = hipStreamSynchronize(g_stream);
    (void)hipFree(staging);
    if (rc || e != hipSuccess) {
        if (!rc) fail("weight repack failed: %s", hipGetErrorString(e));
        (void)hipFree(m->arena);
        delete m;
        return nullptr;
    }
    if (spec->rope_freqs.kind == AOTK_F32) {
        const float *rf = (const float *)((const uint8_t *)blob_host + spec->rope_freqs.off);
        m->rope_freqs.assign(rf, rf + spec->rope_freqs.rows * spec->rope_freqs.cols);
    }
    model_bind(m, map);
    return m;
}

}  // extern "C"

extern "C" {

aotk_model *aotk_model_synthetic(const aotk_model_spec *spec, uint64_t seed) {
    if (ensure_init()) return nullptr;
    if (!spec) {
        fail("aotk_model_synthetic: null spec");
        return nullptr;
    }
    size_t blob_len = 0;
    size_t max_len = 0;
    for_each_tensor(spec, [&](const aotk_tensor &t, uint32_t, bool matrix, bool) {
        size_t len = matrix ? t.len : t.rows * t.cols * 4;
        blob_len = blob_len > t.off + len ? blob_len : t.off + len;
        max_len = max_len > len ? max_len : len;
        return 0;
    });
    if (validate_spec(spec, blob_len)) return nullptr;
    ArenaMap map;
    aotk_model *m = model_alloc(spec, blob_len, map);
    if (!m) return nullptr;
    uint8_t *staging = nullptr;
    if (hipMalloc(&staging, max_len) != hipSuccess) {
        fail("hipMalloc of the %zu-byte synthesis buffer failed", max_len);
        (void)hipFree(m->arena);
        delete m;
        return nullptr;
    }
    for_each_tensor(&m->spec, [&](const aotk_tensor &t, uint32_t idx, bool matrix, bool norm) {
        uint8_t *dst = m->arena + map.find(t.off);
        if (matrix) {
            launch_synth(t.kind, t.rows, t.cols, seed, idx, 0, staging, nullptr, 0, g_stream);
            DevWeight w = dev_weight(m, map, t);
            launch_repack(w, staging, g_stream);
        } else {
            launch_synth(AOTK_F32, 1, t.rows * t.cols, seed, idx, norm ? 1 : 0, dst, nullptr, 0, g_stream);
        }
        return 0;
    });
    hipError_t e = hipStreamSynchronize(g_stream);
    (void)hipFree(staging);
    if (e != hipSuccess) {
        fail("synthesising weights failed: %s", hipGetErrorString(e));
        (void)hipFree(m->arena);
        delete m;
        return nullptr;
    }
    model_bind(m, map);
    return m;
}

int aotk_model_download(const aotk_model *m, void *blob_host, size_t blob_len) {
    if (!m) return fail("null model");
    if (blob_len < m->blob_len) return fail("blob buffer of %zu bytes is smaller than the model's %zu", blob_len, m->blob_len);
    memset(blob_host, 0, blob_len);
    size_t max_len = 0;
    for_each_tensor(&m->spec, [&](const aotk_tensor &t, uint32_t, bool matrix, bool) {
        if (matrix && t.len > max_len) max_len = t.len;
        return 0;
    });
    uint8_t *staging = nullptr;
    HIPC(hipMalloc(&staging, max_len ? max_len : 1));
    ArenaMap map;
    size_t total = 0;
    for_each_tensor(&m->spec, [&](const aotk_tensor &t, uint32_t, bool matrix, bool) {
        if (map.find(t.off) != (size_t)-1) return 0;
        size_t b = matrix ? weight_dev_bytes(t.kind, t.rows, t.cols) : align_up(t.rows * t.cols * 4, 256);
        map.at.push_back({t.off, total});
        total += align_up(b, 256);
        return 0;
    });
    int rc = for_each_tensor(&m->spec, [&](const aotk_tensor &t, uint32_t, bool matrix, bool) {
        uint8_t *dst = (uint8_t *)blob_host + t.off;
        if (matrix) {
            DevWeight w = {};
            w.kind = t.kind;
            w.rows = t.rows;
            w.cols = t.cols;
            weight_set_planes(w, m->arena + map.find(t.off));
            launch_unpack(w, staging, g_stream);
            if (hipMemcpyAsync(dst, staging, t.len, hipMemcpyDeviceToHost, g_stream) != hipSuccess) return -1;
        } else {
            if (hipMemcpyAsync(dst, m->arena + map.find(t.off), t.rows * t.cols * 4, hipMemcpyDeviceToHost, g_stream) != hipSuccess)
                return -1;
        }
        return hipStreamSynchronize(g_stream) == hipSuccess ? 0 : -1;
    });
    (void)hipFree(staging);
    if (rc) return fail("downloading the weights failed");
    return 0;
}

int aotk_model_free(aotk_model *m) {
    if (!m) return 0;
    (void)hipStreamSynchronize(g_stream);
    HIPC(hipFree(m->arena));
    delete m;
    return 0;
}

uint64_t aotk_model_weight_bytes(const aotk_model *m) { return m ? m->weight_bytes : 0; }

}  // extern "C"

// -------------------------------------------------------------------- state

struct aotk_state {
    aotk_model *m;
    size_t ctx, max_batch;
    float *x, *xb, *xb2, *q, *k, *v, *hb, *hb2, *logits;
    float *k_cache, *v_cache;
    ActQ8K ak;
    ActQ8_0 a0;
    float *cs, *cs_local;
    float *attn_ws;
    size_t attn_ws_bytes;
    float *am_ws;
    uint32_t *ctl;     // [0] token, [1] pos, [2] argmax / sampled, [3] generated count, [4] sampler window count
    uint32_t *tokens;  // [max_batch]
    uint32_t *hist;    // [ctx + 1]: a generation from position 0 emits up to ctx + 1 tokens
    uint32_t *ctl_host;  // pinned staging for the control words
    std::vector<void *> allocs;
    // One greedy generation step (argmax, advance, decode step, position
    // increment) captured once as a HIP graph; every kernel of it reads the
    // token and the position from `ctl`, so the same graph serves every step.
    hipGraphExec_t gen_exec = nullptr;
    // Sampling: the token window of the repetition penalty (recent ++
    // generated), the top-k scratch, and the generation step captured for
    // one sampler (its config and rng address are baked into the graph).
    uint32_t *swin = nullptr;  // [ctx + SAMP_WIN_EXTRA]
    uint64_t *samp_ws = nullptr;
    hipGraphExec_t samp_exec = nullptr;
    aotk_sampler_config samp_cfg = {};
    const void *samp_rng = nullptr;
};

// Recent tokens the window keeps beyond the context (repeat_last_n cap).
static constexpr size_t SAMP_WIN_EXTRA = 4096;

struct aotk_sampler {
    aotk_sampler_config cfg;
    uint64_t *rng;  // device
};

static void state_release(aotk_state *st) {
    (void)hipStreamSynchronize(g_stream);
    if (st->gen_exec) (void)hipGraphExecDestroy(st->gen_exec);
    if (st->samp_exec) (void)hipGraphExecDestroy(st->samp_exec);
    for (void *p : st->allocs) (void)hipFree(p);
    if (st->ctl_host) (void)hipHostFree(st->ctl_host);
    delete st;
}

static void rope_table(std::vector<float> &cs, size_t ctx, size_t rot, float base, float scale, const std::vector<float> &ff) {
    // state.rs:308-319 (inv_freq) and ops.rs:28-34 (rope_cos_sin) for every
    // position, on the host with libm, exactly as the reference does per step.
    size_t half = rot / 2;
    std::vector<float> inv(half);
    for (size_t i = 0; i < half; i++) {
        float f = powf(base, -(2.0f * (float)i) / (float)rot);
        if (!ff.empty()) f /= ff[i];
        inv[i] = f;
    }
    cs.assign(ctx * rot, 0.0f);
    for (size_t p = 0; p < ctx; p++) {
        float pos = (float)p / scale;
        for (size_t i = 0; i < half; i++) {
            float a = pos * inv[i];
            cs[p * rot + 2 * i] = cosf(a);
            cs[p * rot + 2 * i + 1] = sinf(a);
        }
    }
}

extern "C" {

aotk_state *aotk_state_new(aotk_model *m, size_t ctx, size_t max_batch) {
    if (!m) {
        fail("null model");
        return nullptr;
    }
    if (ctx == 0 || ctx > 16384) {
        fail("context %zu must be in 1..16384", ctx);
        return nullptr;
    }
    if (max_batch < 1) max_batch = 1;
    const aotk_dims &d = m->spec.dims;
    aotk_state *st = new aotk_state();
    st->m = m;
    st->ctx = ctx;
    st->max_batch = max_batch;
    size_t qd = d.n_head * d.head_dim, kv = d.n_kv_head * d.head_dim;
    size_t nmax = d.dim > qd ? d.dim : qd;
    if (d.hidden > nmax) nmax = d.hidden;
    auto alloc = [&](size_t bytes) -> void * {
        void *p = nullptr;
        if (hipMalloc(&p, bytes ? bytes : 16) != hipSuccess) return nullptr;
        (void)hipMemsetAsync(p, 0, bytes ? bytes : 16, g_stream);
        st->allocs.push_back(p);
        return p;
    };
    size_t B = max_batch;
    bool ok = true;
    auto F = [&](size_t n) -> float * {
        float *p = (float *)alloc(n * 4);
        ok = ok && p;
        return p;
    };
    st->x = F(B * d.dim);
    st->xb = F(B * nmax);
    st->xb2 = F(B * d.dim);
    st->q = F(B * qd);
    st->k = F(B * kv);
    st->v = F(B * kv);
    st->hb = F(B * d.hidden);
    st->hb2 = F(B * d.hidden);
    st->logits = F(d.vocab);
    st->k_cache = F(d.n_layer * ctx * kv);
    st->v_cache = F(d.n_layer * ctx * kv);
    void *ak = alloc(act_q8k_bytes(nmax, B));
    void *a0 = alloc(act_q8_0_bytes(nmax, B));
    ok = ok && ak && a0;
    if (ok) {
        st->ak = act_q8k_view(ak, nmax, B);
        st->a0 = act_q8_0_view(a0, nmax, B);
    }
    st->attn_ws_bytes = attention_scratch_bytes(d.n_head, d.head_dim, ctx, B);
    st->attn_ws = (float *)alloc(st->attn_ws_bytes);
    st->am_ws = F(1024);
    st->ctl = (uint32_t *)alloc(64);
    st->tokens = (uint32_t *)alloc(B * 4);
    st->hist = (uint32_t *)alloc((ctx + 1) * 4);
    st->swin = (uint32_t *)alloc((ctx + SAMP_WIN_EXTRA + 1) * 4);
    st->samp_ws = (uint64_t *)alloc(sampler_scratch_bytes(d.vocab));
    ok = ok && st->attn_ws && st->ctl && st->tokens && st->hist && st->swin && st->samp_ws;
    if (ok && hipHostMalloc((void **)&st->ctl_host, 64, hipHostMallocDefault) != hipSuccess) ok = false;
    // The tables are copied on the library stream, behind the zero fills
    // queued there by alloc() (that stream does not synchronise with the
    // null stream), and each host copy is waited for before it is refilled.
    std::vector<float> cs;
    rope_table(cs, ctx, d.rot_dim, d.rope_base, d.rope_scale, m->rope_freqs);
    st->cs = F(cs.size());
    if (ok) ok = hipMemcpyAsync(st->cs, cs.data(), cs.size() * 4, hipMemcpyHostToDevice, g_stream) == hipSuccess &&
                 hipStreamSynchronize(g_stream) == hipSuccess;
    if (d.swa_window > 0) {
        rope_table(cs, ctx, d.rot_dim, d.rope_base_local, d.rope_scale_local, m->rope_freqs);
        st->cs_local = F(cs.size());
        if (ok) ok = hipMemcpyAsync(st->cs_local, cs.data(), cs.size() * 4, hipMemcpyHostToDevice, g_stream) == hipSuccess &&
                     hipStreamSynchronize(g_stream) == hipSuccess;
    } else {
        st->cs_local = st->cs;
    }
    if (!ok || hipStreamSynchronize(g_stream) != hipSuccess) {
        fail("allocating the state (ctx %zu, batch %zu) failed", ctx, max_batch);
        state_release(st);
        return nullptr;
    }
    return st;
}

int aotk_state_free(aotk_state *st) {
    if (st) state_release(st);
    return 0;
}

}  // extern "C"

// Outputs of an rmsnorm / activation kernel for the consumer kinds (the
// generated code's emit_quantize, emit.rs:131-140).
static RmsOut outs_for(aotk_state *st, std::initializer_list<int> kinds, float *f32) {
    RmsOut o = {};
    for (int k : kinds) {
        int a = activation(k);
        if (a == ACT_F32) o.f32 = f32;
        if (a == ACT_Q8_K) o.q8k = st->ak;
        if (a == ACT_Q8_0) o.q80 = st->a0;
    }
    return o;
}

static const void *act_for(aotk_state *st, int kind, const float *f32) {
    int a = activation(kind);
    if (a == ACT_Q8_K) return &st->ak;
    if (a == ACT_Q8_0) return &st->a0;
    return f32;
}

// The generated layer sequence (emit.rs:243-333 for m == 1, :167-237 for m > 1).
static void run_layers(aotk_state *st, size_t m, size_t pos0, const int *pos_dev) {
    aotk_model *M = st->m;
    const aotk_dims &d = M->spec.dims;
    const aotk_flags &f = M->spec.flags;
    hipStream_t s = g_stream;
    size_t dim = d.dim, qd = d.n_head * d.head_dim, kv = d.n_kv_head * d.head_dim;
    bool normed = false;  // this layer's attention norm done by the previous layer's post-norm join
    for (size_t l = 0; l < d.n_layer; l++) {
        LayerDev &L = M->dev[l];
        float *kc = st->k_cache + l * st->ctx * kv;
        float *vc = st->v_cache + l * st->ctx * kv;
        // attention block
        if (!normed)
            launch_rmsnorm_quant(st->x, L.attn_norm, dim, m, d.eps, outs_for(st, {L.wq.kind, L.wk.kind, L.wv.kind}, st->xb), s);
        normed = false;
        bool same = L.wq.kind == L.wk.kind && L.wk.kind == L.wv.kind && activation(L.wq.kind) != ACT_F32;
        if (same) {
            const DevWeight *ws[3] = {&L.wq, &L.wk, &L.wv};
            float *ys[3] = {st->q, st->k, st->v};
            launch_matvec_multi(3, ws, ys, act_for(st, L.wq.kind, st->xb), m, s);
        } else if (L.wq.kind == L.wk.kind && matvec_pair_ok(L.wq, L.wv)) {
            const DevWeight *ws[2] = {&L.wq, &L.wk};
            float *ys[2] = {st->q, st->k};
            launch_matvec_pair(2, ws, ys, L.wv, st->v, act_for(st, L.wq.kind, st->xb), m, s);
        } else {
            launch_matvec(L.wq, act_for(st, L.wq.kind, st->xb), m, st->q, nullptr, s);
            launch_matvec(L.wk, act_for(st, L.wk.kind, st->xb), m, st->k, nullptr, s);
            launch_matvec(L.wv, act_for(st, L.wv.kind, st->xb), m, st->v, nullptr, s);
        }
        QkvPost p = {};
        p.q = st->q;
        p.k = st->k;
        p.v = st->v;
        p.bq = L.bq;
        p.bk = L.bk;
        p.bv = L.bv;
        p.q_norm = L.q_norm;
        p.k_norm = L.k_norm;
        p.cs = L.local_attn ? st->cs_local : st->cs;
        p.k_cache = kc;
        p.v_cache = vc;
        p.n_head = d.n_head;
        p.n_kv_head = d.n_kv_head;
        p.head_dim = d.head_dim;
        p.rot_dim = d.rot_dim;
        p.neox = f.rope_neox;
        p.eps = d.eps;
        size_t window = L.local_attn ? d.swa_window : 0;
        if (m == 1) {
            launch_attention_decode(st->xb, p, st->ctx, pos0, window, pos_dev, st->attn_ws, s);
        } else {
            launch_qkv_post(p, m, pos0, pos_dev, s);
            launch_attention(st->xb, st->q, kc, vc, d.n_head, d.n_kv_head, d.head_dim, st->ctx, pos0, m, window,
                             pos_dev, st->attn_ws, st->attn_ws_bytes, s);
        }
        // decode: the attention output is quantized inside the wo launch where the kind allows
        float *wo_y = f.post_norms ? st->xb2 : st->x;
        const float *wo_add = f.post_norms ? nullptr : st->x;
        if (!(m == 1 && launch_matvec_quant(L.wo, st->xb, wo_y, wo_add, s))) {
            if (activation(L.wo.kind) != ACT_F32) launch_quant_f32(st->xb, qd, m, outs_for(st, {L.wo.kind}, nullptr), s);
            launch_matvec(L.wo, act_for(st, L.wo.kind, st->xb), m, wo_y, wo_add, s);
        }
        // feed-forward block (Gemma: the post-norm join and the ffn norm in one launch)
        if (f.post_norms)
            launch_rmsnorm_add_quant(st->x, st->xb2, L.attn_post_norm, L.ffn_norm, dim, m, d.eps,
                                     outs_for(st, {L.gate.kind, L.up.kind}, st->xb), s);
        else
            launch_rmsnorm_quant(st->x, L.ffn_norm, dim, m, d.eps, outs_for(st, {L.gate.kind, L.up.kind}, st->xb), s);
        bool same2 = L.gate.kind == L.up.kind && activation(L.gate.kind) != ACT_F32;
        if (same2) {
            const DevWeight *ws[2] = {&L.gate, &L.up};
            float *ys[2] = {st->hb, st->hb2};
            launch_matvec_multi(2, ws, ys, act_for(st, L.gate.kind, st->xb), m, s);
        } else {
            launch_matvec(L.gate, act_for(st, L.gate.kind, st->xb), m, st->hb, nullptr, s);
            launch_matvec(L.up, act_for(st, L.up.kind, st->xb), m, st->hb2, nullptr, s);
        }
        launch_glu_quant(st->hb, st->hb2, d.hidden, m, f.gelu, outs_for(st, {L.down.kind}, st->hb), s);
        if (f.post_norms) {
            launch_matvec(L.down, act_for(st, L.down.kind, st->hb), m, st->xb2, nullptr, s);
            if (l + 1 < d.n_layer) {  // the join and the next layer's attention norm in one launch
                const LayerDev &N = M->dev[l + 1];
                launch_rmsnorm_add_quant(st->x, st->xb2, L.ffn_post_norm, N.attn_norm, dim, m, d.eps,
                                         outs_for(st, {N.wq.kind, N.wk.kind, N.wv.kind}, st->xb), s);
                normed = true;
            } else {
                launch_rmsnorm_add(st->x, st->xb2, L.ffn_post_norm, dim, m, d.eps, s);
            }
        } else {
            launch_matvec(L.down, act_for(st, L.down.kind, st->hb), m, st->x, st->x, s);
        }
    }
}

static void run_logits(aotk_state *st, size_t row) {
    aotk_model *M = st->m;
    const aotk_dims &d = M->spec.dims;
    launch_rmsnorm_quant(st->x + row * d.dim, M->output_norm, d.dim, 1, d.eps, outs_for(st, {M->output.kind}, st->xb), g_stream);
    launch_matvec(M->output, act_for(st, M->output.kind, st->xb), 1, st->logits, nullptr, g_stream);
}

static void run_decode_step(aotk_state *st, int want_logits) {
    aotk_model *M = st->m;
    const aotk_dims &d = M->spec.dims;
    launch_embed(M->embd, st->ctl, 1, sqrtf((float)d.dim), M->spec.flags.embd_scale, st->x, g_stream);
    run_layers(st, 1, 0, (const int *)(st->ctl + 1));
    if (want_logits) run_logits(st, 0);
}

extern "C" {

int aotk_forward(aotk_state *st, uint32_t token, size_t pos, int want_logits) {
    if (!st) return fail("null state");
    const aotk_dims &d = st->m->spec.dims;
    if (token >= d.vocab) return fail("token id %u out of range (vocab %llu)", token, (unsigned long long)d.vocab);
    if (pos >= st->ctx) return fail("position %zu exceeds the context %zu", pos, st->ctx);
    st->ctl_host[0] = token;
    st->ctl_host[1] = (uint32_t)pos;
    HIPC(hipMemcpyAsync(st->ctl, st->ctl_host, 8, hipMemcpyHostToDevice, g_stream));
    run_decode_step(st, want_logits);
    HIPC(hipGetLastError());
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

int aotk_forward_batch(aotk_state *st, const uint32_t *tokens, size_t m, size_t pos0, int want_logits) {
    if (!st) return fail("null state");
    const aotk_dims &d = st->m->spec.dims;
    if (m < 1 || m > st->max_batch) return fail("batch size %zu out of range (max %zu)", m, st->max_batch);
    if (pos0 + m > st->ctx) return fail("positions %zu..%zu exceed the context %zu", pos0, pos0 + m, st->ctx);
    for (size_t i = 0; i < m; i++)
        if (tokens[i] >= d.vocab) return fail("token id %u out of range (vocab %llu)", tokens[i], (unsigned long long)d.vocab);
    HIPC(hipMemcpyAsync(st->tokens, tokens, m * 4, hipMemcpyHostToDevice, g_stream));
    aotk_model *M = st->m;
    launch_embed(M->embd, st->tokens, m, sqrtf((float)d.dim), M->spec.flags.embd_scale, st->x, g_stream);
    run_layers(st, m, pos0, nullptr);
    if (want_logits) run_logits(st, m - 1);
    HIPC(hipGetLastError());
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

int aotk_logits(aotk_state *st, float *out_host) {
    if (!st) return fail("null state");
    HIPC(hipMemcpyAsync(out_host, st->logits, st->m->spec.dims.vocab * 4, hipMemcpyDeviceToHost, g_stream));
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

int aotk_greedy(aotk_state *st, uint32_t *token_out) {
    if (!st) return fail("null state");
    launch_argmax(st->logits, st->m->spec.dims.vocab, st->ctl + 2, st->am_ws, g_stream);
    HIPC(hipGetLastError());
    HIPC(hipMemcpyAsync(st->ctl_host + 2, st->ctl + 2, 4, hipMemcpyDeviceToHost, g_stream));
    HIPC(hipStreamSynchronize(g_stream));
    *token_out = st->ctl_host[2];
    return 0;
}

int aotk_generate_greedy(aotk_state *st, size_t pos, size_t n, uint32_t *tokens_host) {
    if (!st) return fail("null state");
    if (n == 0) return 0;
    if (pos + n - 1 > st->ctx) return fail("generation of %zu tokens from %zu exceeds the context %zu", n, pos, st->ctx);
    const size_t vocab = st->m->spec.dims.vocab;
    st->ctl_host[1] = (uint32_t)pos;
    st->ctl_host[3] = 0;
    HIPC(hipMemcpyAsync(st->ctl + 1, st->ctl_host + 1, 4, hipMemcpyHostToDevice, g_stream));
    HIPC(hipMemcpyAsync(st->ctl + 3, st->ctl_host + 3, 4, hipMemcpyHostToDevice, g_stream));
    auto step = [&]() {
        launch_argmax(st->logits, vocab, st->ctl + 2, st->am_ws, g_stream);
        launch_advance(st->ctl, (int *)(st->ctl + 3), st->hist, st->ctl + 2, g_stream);
        run_decode_step(st, 1);
        launch_inc((int *)(st->ctl + 1), g_stream);
    };
    if (n > 1 && !st->gen_exec && g_decode_graphs) {
        hipGraph_t graph = nullptr;
        HIPC(hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal));
        step();
        hipError_t e = hipStreamEndCapture(g_stream, &graph);
        if (e == hipSuccess) e = hipGraphInstantiate(&st->gen_exec, graph, nullptr, nullptr, 0);
        if (graph) (void)hipGraphDestroy(graph);
        if (e != hipSuccess) {
            st->gen_exec = nullptr;
            return fail("graph capture of the decode step failed: %s", hipGetErrorString(e));
        }
    }
    for (size_t g = 0; g + 1 < n; g++) {
        if (st->gen_exec) HIPC(hipGraphLaunch(st->gen_exec, g_stream));
        else step();
    }
    launch_argmax(st->logits, vocab, st->ctl + 2, st->am_ws, g_stream);
    launch_advance(st->ctl, (int *)(st->ctl + 3), st->hist, st->ctl + 2, g_stream);
    HIPC(hipGetLastError());
    HIPC(hipMemcpyAsync(tokens_host, st->hist, n * 4, hipMemcpyDeviceToHost, g_stream));
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

int aotk_kv_download(aotk_state *st, size_t n_pos, float *k_host, float *v_host) {
    if (!st) return fail("null state");
    const aotk_dims &d = st->m->spec.dims;
    if (n_pos > st->ctx) return fail("n_pos %zu exceeds the context", n_pos);
    size_t kv = d.n_kv_head * d.head_dim;
    for (size_t l = 0; l < d.n_layer; l++) {
        HIPC(hipMemcpyAsync(k_host + l * n_pos * kv, st->k_cache + l * st->ctx * kv, n_pos * kv * 4, hipMemcpyDeviceToHost, g_stream));
        HIPC(hipMemcpyAsync(v_host + l * n_pos * kv, st->v_cache + l * st->ctx * kv, n_pos * kv * 4, hipMemcpyDeviceToHost, g_stream));
    }
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

int aotk_kv_upload(aotk_state *st, size_t n_pos, const float *k_host, const float *v_host) {
    if (!st) return fail("null state");
    const aotk_dims &d = st->m->spec.dims;
    if (n_pos > st->ctx) return fail("n_pos %zu exceeds the context", n_pos);
    size_t kv = d.n_kv_head * d.head_dim;
    for (size_t l = 0; l < d.n_layer; l++) {
        HIPC(hipMemcpyAsync(st->k_cache + l * st->ctx * kv, k_host + l * n_pos * kv, n_pos * kv * 4, hipMemcpyHostToDevice, g_stream));
        HIPC(hipMemcpyAsync(st->v_cache + l * st->ctx * kv, v_host + l * n_pos * kv, n_pos * kv * 4, hipMemcpyHostToDevice, g_stream));
    }
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

// ------------------------------------------------------------- sampling
static uint64_t splitmix_seed(uint64_t seed) {
    // sampler.rs:113-118
    uint64_t z = seed + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return (z ^ (z >> 31)) | 1ull;
}

aotk_sampler *aotk_sampler_new(const aotk_sampler_config *cfg) {
    if (ensure_init()) return nullptr;
    if (!cfg) {
        fail("sampler_new: null config");
        return nullptr;
    }
    if (cfg->repeat_last_n > SAMP_WIN_EXTRA) {
        fail("sampler_new: repeat_last_n %u exceeds %zu", cfg->repeat_last_n, SAMP_WIN_EXTRA);
        return nullptr;
    }
    aotk_sampler *sp = new aotk_sampler();
    sp->cfg = *cfg;
    const uint64_t r = splitmix_seed(cfg->seed);
    if (hipMalloc(&sp->rng, 8) != hipSuccess || hipMemcpy(sp->rng, &r, 8, hipMemcpyHostToDevice) != hipSuccess) {
        fail("sampler_new: device allocation failed");
        if (sp->rng) (void)hipFree(sp->rng);
        delete sp;
        return nullptr;
    }
    return sp;
}

int aotk_sampler_free(aotk_sampler *sp) {
    if (!sp) return 0;
    (void)hipStreamSynchronize(g_stream);
    (void)hipFree(sp->rng);
    delete sp;
    return 0;
}

static int sample_args(aotk_state *st, aotk_sampler *sp, SampleArgs &p) {
    const aotk_sampler_config &c = sp->cfg;
    const size_t V = st->m->spec.dims.vocab;
    const size_t k = c.top_k > 0 ? (c.top_k < V ? c.top_k : V) : V;  // sampler.rs:67
    if (c.temperature > 0.0f && k > (size_t)SAMP_KMAX)
        return fail("sampler: %zu candidates after top-k, at most %d on the device", k, SAMP_KMAX);
    p.logits = st->logits;
    p.vocab = V;
    p.temperature = c.temperature;
    p.top_p = c.top_p;
    p.repeat_penalty = c.repeat_penalty;
    p.repeat_last_n = c.repeat_last_n;
    p.k = (int)k;
    p.rng = sp->rng;
    p.win = st->swin;
    p.count = st->ctl + 4;
    p.tok_out = st->ctl + 2;
    p.scratch = st->samp_ws;
    p.argmax_ws = st->am_ws;
    return 0;
}

// The window starts as the last repeat_last_n tokens of `recent`.
static int upload_window(aotk_state *st, aotk_sampler *sp, const uint32_t *recent, size_t n_recent) {
    const size_t w = n_recent < sp->cfg.repeat_last_n ? n_recent : sp->cfg.repeat_last_n;
    if (w > 0) {
        if (!recent) return fail("sampler: null recent tokens");
        HIPC(hipMemcpyAsync(st->swin, recent + (n_recent - w), w * 4, hipMemcpyHostToDevice, g_stream));
    }
    st->ctl_host[4] = (uint32_t)w;
    HIPC(hipMemcpyAsync(st->ctl + 4, st->ctl_host + 4, 4, hipMemcpyHostToDevice, g_stream));
    return 0;
}

int aotk_set_logits(aotk_state *st, const float *logits_host) {
    if (!st || !logits_host) return fail("set_logits: null argument");
    HIPC(hipMemcpyAsync(st->logits, logits_host, st->m->spec.dims.vocab * 4, hipMemcpyHostToDevice, g_stream));
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

int aotk_sample(aotk_state *st, aotk_sampler *sp, const uint32_t *recent, size_t n_recent, uint32_t *token_out) {
    if (!st || !sp || !token_out) return fail("sample: null argument");
    SampleArgs p;
    if (sample_args(st, sp, p) || upload_window(st, sp, recent, n_recent)) return -1;
    launch_sample(p, g_stream);
    HIPC(hipGetLastError());
    HIPC(hipMemcpyAsync(st->ctl_host + 2, st->ctl + 2, 4, hipMemcpyDeviceToHost, g_stream));
    HIPC(hipStreamSynchronize(g_stream));
    *token_out = st->ctl_host[2];
    return 0;
}

int aotk_generate(aotk_state *st, aotk_sampler *sp, size_t pos, size_t n, const uint32_t *recent, size_t n_recent,
                  uint32_t *tokens_out) {
    if (!st || !sp || (n > 0 && !tokens_out)) return fail("generate: null argument");
    if (n == 0) return 0;
    if (pos + n - 1 > st->ctx) return fail("generation of %zu tokens from %zu exceeds the context %zu", n, pos, st->ctx);
    SampleArgs p;
    if (sample_args(st, sp, p) || upload_window(st, sp, recent, n_recent)) return -1;
    st->ctl_host[1] = (uint32_t)pos;
    st->ctl_host[3] = 0;
    HIPC(hipMemcpyAsync(st->ctl + 1, st->ctl_host + 1, 4, hipMemcpyHostToDevice, g_stream));
    HIPC(hipMemcpyAsync(st->ctl + 3, st->ctl_host + 3, 4, hipMemcpyHostToDevice, g_stream));
    auto pick = [&]() {
        launch_sample(p, g_stream);
        launch_advance(st->ctl, (int *)(st->ctl + 3), st->hist, st->ctl + 2, g_stream);
    };
    auto step = [&]() {
        pick();
        run_decode_step(st, 1);
        launch_inc((int *)(st->ctl + 1), g_stream);
    };
    // the captured step bakes in the sampler's config and rng address
    const bool same = st->samp_exec && st->samp_rng == (const void *)sp->rng &&
                      memcmp(&st->samp_cfg, &sp->cfg, sizeof(sp->cfg)) == 0;
    if (n > 1 && !same && g_decode_graphs) {
        if (st->samp_exec) (void)hipGraphExecDestroy(st->samp_exec);
        st->samp_exec = nullptr;
        hipGraph_t graph = nullptr;
        HIPC(hipStreamBeginCapture(g_stream, hipStreamCaptureModeThreadLocal));
        step();
        hipError_t e = hipStreamEndCapture(g_stream, &graph);
        if (e == hipSuccess) e = hipGraphInstantiate(&st->samp_exec, graph, nullptr, nullptr, 0);
        if (graph) (void)hipGraphDestroy(graph);
        if (e != hipSuccess) {
            st->samp_exec = nullptr;
            return fail("graph capture of the sampling step failed: %s", hipGetErrorString(e));
        }
        st->samp_cfg = sp->cfg;
        st->samp_rng = sp->rng;
    }
    for (size_t g = 0; g + 1 < n; g++) {
        if (st->samp_exec) HIPC(hipGraphLaunch(st->samp_exec, g_stream));
        else step();
    }
    pick();
    HIPC(hipGetLastError());
    HIPC(hipMemcpyAsync(tokens_out, st->hist, n * 4, hipMemcpyDeviceToHost, g_stream));
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

// ------------------------------------------------------ KV prefix blobs
// "AOTP" version 2 (prefix.rs:15-141), little-endian:
//   0 "AOTP" | 4 version | 8 n_tokens | 12 n_layer | 16 kv_dim | 20 n_cached
//   24 token ids u32[n_tokens], zero padding to a 64-byte boundary, then per
//   layer the K rows f32[n_cached * kv_dim] and the V rows likewise.
// Version 1 blobs carry n_cached = n_tokens.
static constexpr size_t PREFIX_HEADER = 24;

static size_t prefix_data_off(size_t n_tokens) { return (PREFIX_HEADER + 4 * n_tokens + 63) / 64 * 64; }

static uint32_t le32_at(const uint8_t *b, size_t at) {
    return (uint32_t)b[at] | ((uint32_t)b[at + 1] << 8) | ((uint32_t)b[at + 2] << 16) | ((uint32_t)b[at + 3] << 24);
}

static void put_le32(uint8_t *b, size_t at, uint32_t v) {
    b[at] = (uint8_t)v;
    b[at + 1] = (uint8_t)(v >> 8);
    b[at + 2] = (uint8_t)(v >> 16);
    b[at + 3] = (uint8_t)(v >> 24);
}

int aotk_prefix_save(aotk_state *st, const uint32_t *tokens, size_t n_tokens, size_t n_cached, void *out, size_t out_cap,
                     size_t *out_len) {
    if (!st || !out_len || (n_tokens > 0 && !tokens)) return fail("prefix_save: null argument");
    const aotk_dims &d = st->m->spec.dims;
    const size_t kv = d.n_kv_head * d.head_dim;
    if (n_cached > n_tokens) n_cached = n_tokens;  // serialize: n_cached.min(n)
    if (n_cached > st->ctx) return fail("prefix_save: %zu cached rows exceed the context %zu", n_cached, st->ctx);
    const size_t off = prefix_data_off(n_tokens);
    const size_t rows = n_cached * kv * 4;
    const size_t len = off + d.n_layer * 2 * rows;
    *out_len = len;
    if (!out) return 0;  // size query
    if (out_cap < len) return fail("prefix_save: buffer of %zu bytes, %zu needed", out_cap, len);
    uint8_t *b = (uint8_t *)out;
    memcpy(b, "AOTP", 4);
    put_le32(b, 4, 2);
    put_le32(b, 8, (uint32_t)n_tokens);
    put_le32(b, 12, (uint32_t)d.n_layer);
    put_le32(b, 16, (uint32_t)kv);
    put_le32(b, 20, (uint32_t)n_cached);
    for (size_t i = 0; i < n_tokens; i++) put_le32(b, PREFIX_HEADER + 4 * i, tokens[i]);
    memset(b + PREFIX_HEADER + 4 * n_tokens, 0, off - PREFIX_HEADER - 4 * n_tokens);
    // the device holds little-endian f32 like the host: rows copy as bytes
    for (size_t l = 0; l < d.n_layer && rows > 0; l++) {
        HIPC(hipMemcpyAsync(b + off + (2 * l) * rows, st->k_cache + l * st->ctx * kv, rows, hipMemcpyDeviceToHost, g_stream));
        HIPC(hipMemcpyAsync(b + off + (2 * l + 1) * rows, st->v_cache + l * st->ctx * kv, rows, hipMemcpyDeviceToHost, g_stream));
    }
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

int aotk_prefix_load(aotk_state *st, const void *blob, size_t len, uint32_t *tokens_out, size_t tokens_cap,
                     size_t *n_tokens, size_t *n_cached) {
    if (!st || (!blob && len > 0) || !n_tokens || !n_cached) return fail("prefix_load: null argument");
    const aotk_dims &d = st->m->spec.dims;
    const size_t kv = d.n_kv_head * d.head_dim;
    const uint8_t *b = (const uint8_t *)blob;
    // Prefix::parse (prefix.rs:48-73): None -> "not a KV cache of this model"
    if (len < PREFIX_HEADER || memcmp(b, "AOTP", 4) != 0) return fail("prefix_load: not a KV prefix blob");
    const uint32_t version = le32_at(b, 4);
    if (version != 1 && version != 2) return fail("prefix_load: unknown version %u", version);
    const size_t n = le32_at(b, 8), nl = le32_at(b, 12), kvd = le32_at(b, 16);
    const size_t nc = version == 1 ? n : le32_at(b, 20);
    if (nl != d.n_layer || kvd != kv || n == 0 || nc > n) return fail("prefix_load: not a KV cache of this model");
    const size_t off = prefix_data_off(n);
    const size_t rows = nc * kv * 4;
    if (len < off + nl * 2 * rows || len < PREFIX_HEADER + 4 * n) return fail("prefix_load: blob truncated");
    if (nc > st->ctx) return fail("prefix_load: %zu cached rows exceed the context %zu", nc, st->ctx);
    *n_tokens = n;
    *n_cached = nc;
    if (tokens_out) {
        if (tokens_cap < n) return fail("prefix_load: room for %zu tokens, %zu needed", tokens_cap, n);
        for (size_t i = 0; i < n; i++) tokens_out[i] = le32_at(b, PREFIX_HEADER + 4 * i);
    }
    // load_into (prefix.rs:96-108): positions 0..n_cached of every layer
    for (size_t l = 0; l < nl && rows > 0; l++) {
        HIPC(hipMemcpyAsync(st->k_cache + l * st->ctx * kv, b + off + (2 * l) * rows, rows, hipMemcpyHostToDevice, g_stream));
        HIPC(hipMemcpyAsync(st->v_cache + l * st->ctx * kv, b + off + (2 * l + 1) * rows, rows, hipMemcpyHostToDevice, g_stream));
    }
    HIPC(hipStreamSynchronize(g_stream));
    return 0;
}

}  // extern "C"

extern "C" {

int aotk_time_matmul(const aotk_weight *const *ws, size_t n_w, const float *xs_dev, size_t m, size_t iters,
                     float *ms_per_launch) {
    if (ensure_init()) return -1;
    if (!ws || n_w == 0 || iters == 0 || m == 0) return fail("time_matmul: nothing to time");
    const DevWeight &w0 = ws[0]->dw;
    for (size_t i = 1; i < n_w; i++)
        if (ws[i]->dw.kind != w0.kind || ws[i]->dw.cols != w0.cols || ws[i]->dw.rows != w0.rows)
            return fail("time_matmul: weights differ in kind or shape");
    int a = activation(w0.kind);
    size_t act_bytes = a == ACT_Q8_K ? act_q8k_bytes(w0.cols, m) : (a == ACT_Q8_0 ? act_q8_0_bytes(w0.cols, m) : 0);
    void *s = lib_scratch(act_bytes + align_up(m * w0.rows * 4, 256));
    if (!s) return -1;
    float *y = (float *)((uint8_t *)s + act_bytes);
    ActQ8K qk;
    ActQ8_0 q0;
    const void *act = xs_dev;
    if (a == ACT_Q8_K) {
        qk = act_q8k_view(s, w0.cols, m);
        launch_quant_q8k(xs_dev, w0.cols, m, qk, g_stream);
        act = &qk;
    } else if (a == ACT_Q8_0) {
        q0 = act_q8_0_view(s, w0.cols, m);
        launch_quant_q8_0(xs_dev, w0.cols, m, q0, g_stream);
        act = &q0;
    }
    hipEvent_t e0, e1;
    HIPC(hipEventCreate(&e0));
    HIPC(hipEventCreate(&e1));
    HIPC(hipEventRecord(e0, g_stream));
    for (size_t it = 0; it < iters; it++) launch_matvec(ws[it % n_w]->dw, act, m, y, nullptr, g_stream);
    HIPC(hipEventRecord(e1, g_stream));
    HIPC(hipEventSynchronize(e1));
    float ms = 0.0f;
    HIPC(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    HIPC(hipGetLastError());
    *ms_per_launch = ms / (float)iters;
    return 0;
}

}  // extern "C"

// HBM ceiling probes: a plain streaming launch of the size under test, no
// grid-stride loop. A block of 256 lanes moves HBM_V * 4 KB: load k of lane t
// reads vector k * 256 + t of the block's range, so every load instruction
// is 1 KB contiguous per wave, and all HBM_V loads are issued before any
// use (HBM_V = 1, 2, 4 or 8 loads in flight per lane). The read probe folds
// what it loaded into one word and stores it (to the library scratch) only
// when that word equals one constant, so the loads cannot be dropped and
// nothing else is written. Its loads carry the nontemporal hint, as the
// decode matvecs' weight loads do (cold 33 MB reads 6.86 -> 6.68 us).
typedef unsigned hbm_u4 __attribute__((ext_vector_type(4)));
template <int HBM_V>
__global__ __launch_bounds__(256) void k_hbm_read(const uint4 *src, size_t n16, uint32_t *sink) {
    const size_t base = (size_t)blockIdx.x * 256 * HBM_V + threadIdx.x;
    uint4 v[HBM_V];
#pragma unroll
    for (int k = 0; k < HBM_V; k++) {
        const hbm_u4 t = base + k * 256 < n16 ? __builtin_nontemporal_load((const hbm_u4 *)(src + base + k * 256)) : hbm_u4{0, 0, 0, 0};
        v[k] = make_uint4(t.x, t.y, t.z, t.w);
    }
    uint32_t acc = 0;
#pragma unroll
    for (int k = 0; k < HBM_V; k++) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    if (acc == 0x9E3779B9u && base == 0) sink[0] = acc;
}
template <int HBM_V>
__global__ __launch_bounds__(256) void k_hbm_copy(uint4 *dst, const uint4 *src, size_t n16) {
    const size_t base = (size_t)blockIdx.x * 256 * HBM_V + threadIdx.x;
    uint4 v[HBM_V];
#pragma unroll
    for (int k = 0; k < HBM_V; k++)
        if (base + k * 256 < n16) v[k] = src[base + k * 256];
#pragma unroll
    for (int k = 0; k < HBM_V; k++)
        if (base + k * 256 < n16) dst[base + k * 256] = v[k];
}

extern "C" {

int aotk_time_hbm(int copy, int loads_per_lane, void *const *bufs, size_t n_bufs, size_t bytes, size_t iters,
                  float *ms_per_launch) {
    if (ensure_init()) return -1;
    const int U = loads_per_lane;
    if (U != 1 && U != 2 && U != 4 && U != 8) return fail("time_hbm: loads_per_lane must be 1, 2, 4 or 8");
    if (!bufs || n_bufs < (copy ? 2u : 1u) || iters == 0 || bytes < 16 || bytes % 16)
        return fail("time_hbm: need %s buffer(s), iters > 0 and a size that is a multiple of 16 bytes", copy ? "2+" : "1+");
    for (size_t i = 0; i < n_bufs; i++)
        if (!bufs[i] || ((uintptr_t)bufs[i] & 15)) return fail("time_hbm: buffer %zu is null or not 16-byte aligned", i);
    const size_t n16 = bytes / 16;
    const size_t blocks = (n16 + 256 * (size_t)U - 1) / (256 * (size_t)U);
    if (blocks > 0x7fffffffu) return fail("time_hbm: %zu bytes is too large", bytes);
    uint32_t *sink = (uint32_t *)lib_scratch(256);
    if (!sink) return -1;
    auto one = [&](size_t it) {
        const unsigned g = (unsigned)blocks;
        uint4 *d = (uint4 *)bufs[(it + 1) % n_bufs];
        const uint4 *src = (const uint4 *)bufs[it % n_bufs];
        if (copy) {
            switch (U) {
            case 1: k_hbm_copy<1><<<g, 256, 0, g_stream>>>(d, src, n16); break;
            case 2: k_hbm_copy<2><<<g, 256, 0, g_stream>>>(d, src, n16); break;
            case 4: k_hbm_copy<4><<<g, 256, 0, g_stream>>>(d, src, n16); break;
            default: k_hbm_copy<8><<<g, 256, 0, g_stream>>>(d, src, n16); break;
            }
        } else {
            switch (U) {
            case 1: k_hbm_read<1><<<g, 256, 0, g_stream>>>(src, n16, sink); break;
            case 2: k_hbm_read<2><<<g, 256, 0, g_stream>>>(src, n16, sink); break;
            case 4: k_hbm_read<4><<<g, 256, 0, g_stream>>>(src, n16, sink); break;
            default: k_hbm_read<8><<<g, 256, 0, g_stream>>>(src, n16, sink); break;
            }
        }
    };
    one(0);  // warm-up
    hipEvent_t e0, e1;
    HIPC(hipEventCreate(&e0));
    HIPC(hipEventCreate(&e1));
    HIPC(hipEventRecord(e0, g_stream));
    for (size_t it = 0; it < iters; it++) one(it);
    HIPC(hipEventRecord(e1, g_stream));
    HIPC(hipEventSynchronize(e1));
    float ms = 0.0f;
    HIPC(hipEventElapsedTime(&ms, e0, e1));
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    HIPC(hipGetLastError());
    *ms_per_launch = ms / (float)iters;
    return 0;
}

int aotk_time_matvec(const aotk_weight *const *ws, size_t n_w, const float *x_dev, size_t iters, float *ms_per_launch) {
    return aotk_time_matmul(ws, n_w, x_dev, 1, iters, ms_per_launch);
}

}  // extern "C"
