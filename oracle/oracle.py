"""ctypes binding of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker / CPU baseline, never by the
product path (aot-llm_amd/).
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

Q8_0_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", 32)])
Q8_K_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bsums", "<i2", 16)])
assert Q8_0_DTYPE.itemsize == 36 and Q8_K_DTYPE.itemsize == 292

_lib = None


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
    lib = C.CDLL(LIB_PATH)
    vp, sz, i, f, u32, u64 = C.c_void_p, C.c_size_t, C.c_int, C.c_float, C.c_uint32, C.c_uint64

    def sig(name, res, args):
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args

    sig("or_f16_to_f32", f, [C.c_uint16])
    sig("or_f32_to_f16", C.c_uint16, [f])
    sig("or_bf16_to_f32", f, [C.c_uint16])
    sig("or_f32_to_bf16", C.c_uint16, [f])
    sig("or_row_bytes", sz, [i, sz])
    sig("or_quantize_q8_0", None, [vp, sz, vp])
    sig("or_quantize_q8_k", None, [vp, sz, vp])
    sig("or_dequant_row", None, [i, vp, vp, sz])
    sig("or_quantize_row", sz, [i, vp, sz, vp])
    sig("or_dot_scalar", f, [i, vp, vp, sz])
    sig("or_dot_avx2", f, [i, vp, vp, sz])
    sig("or_dot_avx2_x4", i, [i, vp, C.POINTER(vp), sz, C.POINTER(f)])
    sig("or_pool_new", vp, [i])
    sig("or_pool_free", None, [vp])
    sig("or_matvec", None, [vp, i, i, vp, vp, vp, sz, sz])
    sig("or_matmul", None, [vp, i, i, vp, vp, vp, sz, sz, sz])
    sig("or_rmsnorm", None, [vp, vp, vp, sz, f])
    sig("or_rope_cos_sin", None, [vp, vp, sz, f])
    sig("or_rope", None, [vp, sz, sz, sz, vp, i])
    sig("or_rmsnorm_heads", None, [vp, vp, sz, sz, f])
    sig("or_softmax", None, [vp, sz])
    sig("or_silu_mul", None, [vp, vp, sz])
    sig("or_gelu", f, [f])
    sig("or_gelu_mul", None, [vp, vp, sz])
    sig("or_window_start", sz, [sz, sz])
    sig("or_sampler_seed", u64, [u64])
    sig("or_sample", u32, [vp, C.POINTER(u64), vp, sz, vp, sz])
    sig("or_attention", None, [vp, vp, vp, vp, vp, sz, sz, sz, sz, sz, sz, sz, sz])
    sig("or_inv_freq", None, [vp, sz, f, vp])
    sig("or_argmax", u32, [vp, sz])
    sig("or_synth_value", f, [u64, u32, u64])
    sig("or_synth_blob", i, [vp, u64, vp, sz, i])
    sig("or_e2e_uniform", None, [C.POINTER(u64), f, vp, sz])
    sig("or_model_new", vp, [vp, vp, sz, sz, sz, i, i])
    sig("or_model_free", None, [vp])
    sig("or_forward", i, [vp, u32, sz, i])
    sig("or_forward_batch", i, [vp, C.POINTER(u32), sz, sz, i])
    sig("or_logits", C.POINTER(f), [vp])
    sig("or_k_cache", C.POINTER(f), [vp])
    sig("or_v_cache", C.POINTER(f), [vp])
    _lib = lib
    return lib


def ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def quantize_q8_0(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.size // 32, Q8_0_DTYPE)
    load().or_quantize_q8_0(ptr(x), x.size, ptr(out))
    return out


def quantize_q8_k(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros(x.size // 256, Q8_K_DTYPE)
    load().or_quantize_q8_k(ptr(x), x.size, ptr(out))
    return out


def quantize_act(kind, x):
    """Activation for a matrix of `kind` (model.rs:85-91)."""
    if kind in (3, 4, 5):
        return quantize_q8_0(x)
    if kind in (6, 7, 8):
        return quantize_q8_k(x)
    return np.ascontiguousarray(x, np.float32)


def row_bytes(kind, cols):
    return load().or_row_bytes(kind, cols)


def quantize_rows(kind, x):
    """quantize.rs:282-294 over each row of a 2-D array -> uint8 [rows, rb]."""
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    rb = row_bytes(kind, cols)
    out = np.zeros((rows, rb), np.uint8)
    lib = load()
    for r in range(rows):
        lib.or_quantize_row(kind, ptr(x[r]), cols, ptr(out[r]))
    return out


def dequant_rows(kind, w, cols):
    w = np.ascontiguousarray(w, np.uint8).reshape(-1, row_bytes(kind, cols))
    out = np.zeros((w.shape[0], cols), np.float32)
    lib = load()
    for r in range(w.shape[0]):
        lib.or_dequant_row(kind, ptr(w[r]), ptr(out[r]), cols)
    return out


def dot(kind, w_row, x, cols, kernels="avx2"):
    lib = load()
    fn = lib.or_dot_avx2 if kernels == "avx2" else lib.or_dot_scalar
    return fn(kind, ptr(np.ascontiguousarray(w_row)), ptr(x), cols)


class Pool:
    def __init__(self, n):
        self.p = load().or_pool_new(n)

    def __del__(self):
        if getattr(self, "p", None):
            load().or_pool_free(self.p)
            self.p = None


def matvec(kind, w, x, rows, cols, pool=None, kernels=1):
    out = np.zeros(rows, np.float32)
    load().or_matvec(pool.p if pool else None, kernels, kind, ptr(out), ptr(np.ascontiguousarray(w)), ptr(x), rows, cols)
    return out


def matmul(kind, w, xs, m, rows, cols, pool=None, kernels=1):
    out = np.zeros(m * rows, np.float32)
    load().or_matmul(pool.p if pool else None, kernels, kind, ptr(out), ptr(np.ascontiguousarray(w)), ptr(xs), m, rows, cols)
    return out


def synth_blob(spec, seed, n_threads=8):
    blob = np.zeros(spec.blob_len, np.uint8)
    rc = load().or_synth_blob(C.cast(spec.ptr(), C.c_void_p), seed, ptr(blob), blob.size, n_threads)
    if rc != 0:
        raise RuntimeError("or_synth_blob failed")
    return blob


class Model:
    """The CPU reference model (emitted forward / forward_batch)."""

    def __init__(self, spec, blob, ctx, max_batch=64, n_threads=8, kernels=1):
        self.spec = spec
        self.blob = blob  # keep alive
        self.vocab = spec.d["vocab"]
        self.m = load().or_model_new(C.cast(spec.ptr(), C.c_void_p), ptr(blob), blob.size, ctx, max_batch, n_threads, kernels)

    def forward(self, token, pos, want_logits=True):
        if load().or_forward(self.m, token, pos, 1 if want_logits else 0) != 0:
            raise ValueError("or_forward: token or position out of range")

    def forward_batch(self, tokens, pos0, want_logits=True):
        arr = (C.c_uint32 * len(tokens))(*tokens)
        if load().or_forward_batch(self.m, arr, len(tokens), pos0, 1 if want_logits else 0) != 0:
            raise ValueError("or_forward_batch: bad batch")

    def logits(self):
        p = load().or_logits(self.m)
        return np.ctypeslib.as_array(p, (self.vocab,)).copy()

    def kv(self, ctx):
        d = self.spec.d
        n = d["n_layer"] * ctx * d["n_kv_head"] * d["head_dim"]
        k = np.ctypeslib.as_array(load().or_k_cache(self.m), (n,))
        v = np.ctypeslib.as_array(load().or_v_cache(self.m), (n,))
        return k, v

    def prompt(self, tokens, batch=64):
        """app.rs:474-485: chunks of `batch`, a chunk of 1 uses forward."""
        done = 0
        while done < len(tokens):
            end = min(done + batch, len(tokens))
            last = end == len(tokens)
            if end - done == 1:
                self.forward(tokens[done], done, last)
            else:
                self.forward_batch(tokens[done:end], done, last)
            done = end

    def generate(self, pos, n):
        """Greedy loop of app.rs:553-610 (temperature 0): returns n ids."""
        out = []
        for g in range(n):
            t = argmax(self.logits())
            out.append(t)
            if g + 1 < n:
                self.forward(t, pos, True)
                pos += 1
        return out

    def generate_sampled(self, pos, n, sampler, recent):
        """The app.rs:553-610 loop with a sampler: `recent` = the tokens so
        far (prompt), extended by every sampled token."""
        all_toks = list(recent)
        out = []
        for g in range(n):
            lg = self.logits()
            t = sampler.sample(lg, all_toks)
            out.append(t)
            all_toks.append(t)
            if g + 1 < n:
                self.forward(t, pos, True)
                pos += 1
        return out

    def close(self):
        if self.m:
            load().or_model_free(self.m)
            self.m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def argmax(x):
    x = np.ascontiguousarray(x, np.float32)
    return int(load().or_argmax(ptr(x), x.size))


class SamplerConfig(C.Structure):
    """aotk_sampler_config / sampler.rs SamplerConfig."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_uint32), ("top_p", C.c_float), ("repeat_penalty", C.c_float),
                ("repeat_last_n", C.c_uint32), ("reserved", C.c_uint32), ("seed", C.c_uint64)]


class Sampler:
    """sampler.rs Sampler: the config and the xorshift64* state."""

    def __init__(self, temperature=0.0, top_k=40, top_p=0.95, repeat_penalty=1.0, repeat_last_n=64, seed=42):
        self.cfg = SamplerConfig(temperature, top_k, top_p, repeat_penalty, repeat_last_n, 0, seed)
        self.rng = C.c_uint64(load().or_sampler_seed(seed))

    def sample(self, logits, recent=()):
        """Sampler::sample; `logits` (float32 array) is modified in place."""
        assert logits.dtype == np.float32 and logits.flags.c_contiguous
        rec = np.ascontiguousarray(np.asarray(recent, np.uint32))
        return int(load().or_sample(C.byref(self.cfg), C.byref(self.rng), ptr(logits), logits.size,
                                    ptr(rec) if rec.size else None, rec.size))


# ----------------------------------------------------------- KV prefix blobs
# Restatement of crates/aot-kernels/src/prefix.rs (format comment :15-26):
# "AOTP", version, n_tokens, n_layer, kv_dim, n_cached (u32 LE each), the
# token ids, zero padding to 64 bytes, then per layer K rows and V rows f32.
PREFIX_MAGIC = b"AOTP"


def prefix_serialize(k_cache, v_cache, ctx, n_layer, kv_dim, tokens, n_cached):
    """prefix::serialize (prefix.rs:114-141); k_cache / v_cache laid out
    [n_layer][ctx][kv_dim] like State::k_cache."""
    n = len(tokens)
    n_cached = min(n_cached, n)  # :117
    out = bytearray()
    out += PREFIX_MAGIC
    out += np.array([2, n, n_layer, kv_dim, n_cached], "<u4").tobytes()  # :120-125
    out += np.asarray(tokens, "<u4").tobytes()  # :126-128
    while len(out) % 64:  # :129-131
        out.append(0)
    k = np.asarray(k_cache, "<f4").reshape(n_layer, ctx, kv_dim)
    v = np.asarray(v_cache, "<f4").reshape(n_layer, ctx, kv_dim)
    for layer in range(n_layer):  # :132-139
        out += k[layer, :n_cached].tobytes()
        out += v[layer, :n_cached].tobytes()
    return bytes(out)


def prefix_parse(blob, n_layer, kv_dim):
    """Prefix::parse (prefix.rs:48-73): (tokens, n_cached, k_rows, v_rows)
    with rows [n_layer][n_cached][kv_dim], or None where the reference
    returns None."""
    if len(blob) < 24 or blob[:4] != PREFIX_MAGIC:
        return None
    version, n, nl, kvd, nc = np.frombuffer(blob[4:24], "<u4").tolist()
    if version not in (1, 2):
        return None
    if version == 1:
        nc = n
    if nl != n_layer or kvd != kv_dim or n == 0 or nc > n:
        return None
    tokens = np.frombuffer(blob[24:24 + 4 * n], "<u4").tolist()
    off = (24 + 4 * n + 63) // 64 * 64
    need = off + nl * 2 * nc * kvd * 4
    if len(blob) < need:
        return None
    data = np.frombuffer(blob[off:need], "<f4").reshape(nl, 2, nc, kvd)
    return tokens, nc, data[:, 0].copy(), data[:, 1].copy()
