"""Python wrappers over the C ABI (include/aotk.h), with numpy host arrays."""
import ctypes as C

import numpy as np

from . import abi

Q8_0_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", 32)])
Q8_K_DTYPE = np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bsums", "<i2", 16)])


def _lib():
    return abi.load()


def init(device=0):
    abi.check(_lib().aotk_init(device))


def sync():
    abi.check(_lib().aotk_sync())


def stream():
    return _lib().aotk_stream()


def _np_ptr(a):
    return a.ctypes.data_as(C.c_void_p)


def copy_dev(dst, src, nbytes):
    """Device-to-device copy of `nbytes` between DeviceBuffers (synchronous)."""
    assert nbytes <= dst.nbytes and nbytes <= src.nbytes
    abi.check(_lib().aotk_d2d(dst.ptr, src.ptr, nbytes))


class DeviceBuffer:
    """A device allocation owned by Python."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = abi.check_ptr(_lib().aotk_dev_alloc(self.nbytes))

    @classmethod
    def from_numpy(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        if a.nbytes:
            abi.check(_lib().aotk_h2d(b.ptr, _np_ptr(a), a.nbytes))
        return b

    def to_numpy(self, dtype, count=None):
        dtype = np.dtype(dtype)
        n = self.nbytes // dtype.itemsize if count is None else count
        out = np.empty(n, dtype)
        if out.nbytes:
            abi.check(_lib().aotk_d2h(_np_ptr(out), self.ptr, out.nbytes))
        return out

    def upload(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        abi.check(_lib().aotk_h2d(self.ptr, _np_ptr(a), a.nbytes))

    def free(self):
        if self.ptr:
            _lib().aotk_dev_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Weight:
    """A quantized matrix resident in HBM (`w: &[u8]` of matvec_*)."""

    def __init__(self, kind, raw, rows, cols):
        raw = np.ascontiguousarray(raw, np.uint8)
        assert raw.size == rows * abi.row_bytes(kind, cols), "raw bytes do not match rows * row_bytes"
        self.kind, self.rows, self.cols = kind, rows, cols
        self.h = abi.check_ptr(_lib().aotk_weight_upload(kind, _np_ptr(raw), rows, cols))

    def free(self):
        if self.h:
            _lib().aotk_weight_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def time_hbm(buffers, nbytes, iters, copy=False, loads_per_lane=4):
    """Mean ms per launch of the HBM probe (read-only, or a copy from each
    buffer to the next) over `nbytes` of the DeviceBuffers in turn."""
    arr = (C.c_void_p * len(buffers))(*[b.ptr for b in buffers])
    for b in buffers:
        assert nbytes <= b.nbytes
    ms = C.c_float()
    abi.check(_lib().aotk_time_hbm(1 if copy else 0, int(loads_per_lane), arr, len(buffers), int(nbytes), int(iters), C.byref(ms)))
    return ms.value


def time_matvec(weights, x, iters):
    """Mean device ms per matvec launch, rotating over `weights` (same kind
    and shape), timed with HIP events on the library stream."""
    dx = DeviceBuffer.from_numpy(np.ascontiguousarray(x, np.float32))
    arr = (C.c_void_p * len(weights))(*[w.h for w in weights])
    ms = C.c_float()
    abi.check(_lib().aotk_time_matvec(arr, len(weights), dx.ptr, iters, C.byref(ms)))
    return ms.value


def time_matmul(weights, xs, iters):
    """Mean device ms per batched product of the m rows of `xs` (m x cols
    f32, quantized once on the device), rotating over `weights`."""
    xs = np.ascontiguousarray(xs, np.float32)
    dx = DeviceBuffer.from_numpy(xs)
    arr = (C.c_void_p * len(weights))(*[w.h for w in weights])
    ms = C.c_float()
    abi.check(_lib().aotk_time_matmul(arr, len(weights), dx.ptr, xs.shape[0], iters, C.byref(ms)))
    return ms.value


def dequant_rows(w, row0=0, n_rows=None):
    n_rows = w.rows - row0 if n_rows is None else n_rows
    out = DeviceBuffer(n_rows * w.cols * 4)
    abi.check(_lib().aotk_dequant_rows(w.h, row0, n_rows, out.ptr))
    return out.to_numpy(np.float32).reshape(n_rows, w.cols)


def quantize_rows(kind, x):
    """Reference weight encoders on the device (quantize.rs:282-294)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    dx = DeviceBuffer.from_numpy(x)
    out = DeviceBuffer(rows * abi.row_bytes(kind, cols))
    abi.check(_lib().aotk_quantize_rows(kind, dx.ptr, rows, cols, out.ptr))
    return out.to_numpy(np.uint8).reshape(rows, -1)


def quantize_q8_0(x):
    x = np.ascontiguousarray(x, np.float32)
    dx = DeviceBuffer.from_numpy(x)
    out = DeviceBuffer(x.size // 32 * 36)
    abi.check(_lib().aotk_quantize_q8_0(dx.ptr, x.size, out.ptr))
    return out.to_numpy(Q8_0_DTYPE)


def quantize_q8_k(x):
    x = np.ascontiguousarray(x, np.float32)
    dx = DeviceBuffer.from_numpy(x)
    out = DeviceBuffer(x.size // 256 * 292)
    abi.check(_lib().aotk_quantize_q8_k(dx.ptr, x.size, out.ptr))
    return out.to_numpy(Q8_K_DTYPE)


def matvec(w, x_act):
    """`matvec_<kind>` with a pre-quantized input (Q8_0/Q8_K blocks or f32)."""
    dx = DeviceBuffer.from_numpy(np.ascontiguousarray(x_act))
    out = DeviceBuffer(w.rows * 4)
    abi.check(_lib().aotk_matvec(w.h, dx.ptr, out.ptr))
    return out.to_numpy(np.float32)


def matmul(w, xs_act, m):
    dx = DeviceBuffer.from_numpy(np.ascontiguousarray(xs_act))
    out = DeviceBuffer(m * w.rows * 4)
    abi.check(_lib().aotk_matmul(w.h, dx.ptr, m, out.ptr))
    return out.to_numpy(np.float32).reshape(m, w.rows)


def matvec3(ws, x_act):
    """matvec3_*_input (matvec.rs:321-355): three matrices of one kind and
    width over one pre-quantized input, one launch."""
    dx = DeviceBuffer.from_numpy(np.ascontiguousarray(x_act))
    outs = [DeviceBuffer(w.rows * 4) for w in ws]
    warr = (C.c_void_p * 3)(*[w.h for w in ws])
    oarr = (C.c_void_p * 3)(*[o.ptr for o in outs])
    abi.check(_lib().aotk_matvec3(warr, dx.ptr, oarr))
    return [o.to_numpy(np.float32) for o in outs]


def matvec2(wa, wb, x_act):
    """matvec2_*_input (matvec.rs:403-439): the gate/up pair."""
    dx = DeviceBuffer.from_numpy(np.ascontiguousarray(x_act))
    oa, ob = DeviceBuffer(wa.rows * 4), DeviceBuffer(wb.rows * 4)
    abi.check(_lib().aotk_matvec2(wa.h, wb.h, dx.ptr, oa.ptr, ob.ptr))
    return oa.to_numpy(np.float32), ob.to_numpy(np.float32)


def matmul2(wa, wb, xs_act, m):
    """matmul2_*_input (matvec.rs:569-583): the batched gate/up pair."""
    dx = DeviceBuffer.from_numpy(np.ascontiguousarray(xs_act))
    oa, ob = DeviceBuffer(m * wa.rows * 4), DeviceBuffer(m * wb.rows * 4)
    abi.check(_lib().aotk_matmul2(wa.h, wb.h, dx.ptr, m, oa.ptr, ob.ptr))
    return oa.to_numpy(np.float32).reshape(m, wa.rows), ob.to_numpy(np.float32).reshape(m, wb.rows)


def matmul_noalloc(w, xs_act, m):
    """aotk_matmul_noalloc: the same product staged in the library's fixed
    device array (the caller's buffers are allocated here, the call itself
    allocates nothing)."""
    dx = DeviceBuffer.from_numpy(np.ascontiguousarray(xs_act))
    out = DeviceBuffer(m * w.rows * 4)
    abi.check(_lib().aotk_matmul_noalloc(w.h, dx.ptr, m, out.ptr))
    return out.to_numpy(np.float32).reshape(m, w.rows)


def matvec_f32(w, x):
    dx = DeviceBuffer.from_numpy(np.ascontiguousarray(x, np.float32))
    out = DeviceBuffer(w.rows * 4)
    abi.check(_lib().aotk_matvec_f32(w.h, dx.ptr, out.ptr))
    return out.to_numpy(np.float32)


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    m, n = (1, x.size) if x.ndim == 1 else x.shape
    dx, dw, out = DeviceBuffer.from_numpy(x), DeviceBuffer.from_numpy(np.asarray(w, np.float32)), DeviceBuffer(x.nbytes)
    abi.check(_lib().aotk_rmsnorm(out.ptr, dx.ptr, dw.ptr, n, m, eps))
    return out.to_numpy(np.float32).reshape(x.shape)


def rmsnorm_heads(x, w, n_heads, head_dim, eps):
    dx, dw = DeviceBuffer.from_numpy(np.asarray(x, np.float32)), DeviceBuffer.from_numpy(np.asarray(w, np.float32))
    abi.check(_lib().aotk_rmsnorm_heads(dx.ptr, dw.ptr, n_heads, head_dim, eps))
    return dx.to_numpy(np.float32)


def rope(x, m, n_heads, head_dim, rot_dim, cs, neox):
    dx, dc = DeviceBuffer.from_numpy(np.asarray(x, np.float32)), DeviceBuffer.from_numpy(np.asarray(cs, np.float32))
    abi.check(_lib().aotk_rope(dx.ptr, m, n_heads, head_dim, rot_dim, dc.ptr, 1 if neox else 0))
    return dx.to_numpy(np.float32)


def softmax(x):
    dx = DeviceBuffer.from_numpy(np.asarray(x, np.float32))
    abi.check(_lib().aotk_softmax(dx.ptr, dx.nbytes // 4))
    return dx.to_numpy(np.float32)


def silu_mul(h, up):
    dh, du = DeviceBuffer.from_numpy(np.asarray(h, np.float32)), DeviceBuffer.from_numpy(np.asarray(up, np.float32))
    abi.check(_lib().aotk_silu_mul(dh.ptr, du.ptr, dh.nbytes // 4))
    return dh.to_numpy(np.float32)


def gelu_mul(h, up):
    dh, du = DeviceBuffer.from_numpy(np.asarray(h, np.float32)), DeviceBuffer.from_numpy(np.asarray(up, np.float32))
    abi.check(_lib().aotk_gelu_mul(dh.ptr, du.ptr, dh.nbytes // 4))
    return dh.to_numpy(np.float32)


def attention(q, k_cache, v_cache, n_head, n_kv_head, head_dim, ctx, layer, pos0, m, window):
    dq = DeviceBuffer.from_numpy(np.asarray(q, np.float32))
    dk = DeviceBuffer.from_numpy(np.asarray(k_cache, np.float32))
    dv = DeviceBuffer.from_numpy(np.asarray(v_cache, np.float32))
    out = DeviceBuffer(m * n_head * head_dim * 4)
    abi.check(_lib().aotk_attention(out.ptr, dq.ptr, dk.ptr, dv.ptr, n_head, n_kv_head, head_dim, ctx, layer, pos0, m, window))
    return out.to_numpy(np.float32)


def argmax(x):
    dx = DeviceBuffer.from_numpy(np.asarray(x, np.float32))
    out = C.c_uint32()
    abi.check(_lib().aotk_argmax(dx.ptr, dx.nbytes // 4, C.byref(out)))
    return out.value


class Model:
    """Weights resident in HBM, uploaded once (`aotk_model_load`) or built on
    the device from the synthetic generator (`aotk_model_synthetic`)."""

    def __init__(self, spec, blob=None, seed=None):
        self.spec = spec
        lib = _lib()
        if blob is not None:
            blob = np.ascontiguousarray(blob, np.uint8)
            self.h = abi.check_ptr(lib.aotk_model_load(spec.ptr(), _np_ptr(blob), blob.size))
        else:
            self.h = abi.check_ptr(lib.aotk_model_synthetic(spec.ptr(), int(seed)))

    def download(self):
        blob = np.zeros(self.spec.blob_len, np.uint8)
        abi.check(_lib().aotk_model_download(self.h, _np_ptr(blob), blob.size))
        return blob

    def weight_bytes(self):
        return int(_lib().aotk_model_weight_bytes(self.h))

    def free(self):
        if self.h:
            _lib().aotk_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Sampler:
    """sampler.rs Sampler on the device: the config and the xorshift64* state
    (seeded through splitmix) live in the library."""

    def __init__(self, temperature=0.0, top_k=40, top_p=0.95, repeat_penalty=1.0, repeat_last_n=64, seed=42):
        self.cfg = abi.SamplerConfig(temperature, top_k, top_p, repeat_penalty, repeat_last_n, 0, seed)
        self.h = abi.check_ptr(_lib().aotk_sampler_new(C.byref(self.cfg)))

    def free(self):
        if self.h:
            _lib().aotk_sampler_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _u32_array(xs):
    xs = [int(x) for x in xs]
    return (C.c_uint32 * max(1, len(xs)))(*xs), len(xs)


class State:
    """Activations + KV cache in HBM for one sequence (state.rs:251-355)."""

    def __init__(self, model, ctx, max_batch=64):
        self.model = model
        self.ctx = ctx
        self.vocab = model.spec.d["vocab"]
        self.h = abi.check_ptr(_lib().aotk_state_new(model.h, ctx, max_batch))

    def forward(self, token, pos, want_logits=True):
        abi.check(_lib().aotk_forward(self.h, int(token), int(pos), 1 if want_logits else 0))

    def forward_batch(self, tokens, pos0, want_logits=True):
        arr = (C.c_uint32 * len(tokens))(*[int(t) for t in tokens])
        abi.check(_lib().aotk_forward_batch(self.h, arr, len(tokens), int(pos0), 1 if want_logits else 0))

    def prompt(self, tokens, batch=64):
        """app.rs:474-485: chunks of `batch`; a chunk of one token uses forward."""
        done = 0
        while done < len(tokens):
            end = min(done + batch, len(tokens))
            last = end == len(tokens)
            if end - done == 1:
                self.forward(tokens[done], done, last)
            else:
                self.forward_batch(tokens[done:end], done, last)
            done = end

    def logits(self):
        out = np.empty(self.vocab, np.float32)
        abi.check(_lib().aotk_logits(self.h, out.ctypes.data_as(C.POINTER(C.c_float))))
        return out

    def greedy(self):
        t = C.c_uint32()
        abi.check(_lib().aotk_greedy(self.h, C.byref(t)))
        return t.value

    def generate(self, pos, n):
        out = (C.c_uint32 * n)()
        abi.check(_lib().aotk_generate_greedy(self.h, int(pos), int(n), out))
        return list(out)

    def kv_download(self, n_pos):
        d = self.model.spec.d
        n = d["n_layer"] * n_pos * d["n_kv_head"] * d["head_dim"]
        k = np.empty(n, np.float32)
        v = np.empty(n, np.float32)
        fp = C.POINTER(C.c_float)
        abi.check(_lib().aotk_kv_download(self.h, n_pos, k.ctypes.data_as(fp), v.ctypes.data_as(fp)))
        return k, v

    def kv_upload(self, n_pos, k, v):
        fp = C.POINTER(C.c_float)
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        abi.check(_lib().aotk_kv_upload(self.h, n_pos, k.ctypes.data_as(fp), v.ctypes.data_as(fp)))

    def set_logits(self, logits):
        x = np.ascontiguousarray(logits, np.float32)
        assert x.size == self.vocab
        abi.check(_lib().aotk_set_logits(self.h, x.ctypes.data_as(C.POINTER(C.c_float))))

    def sample(self, sampler, recent=()):
        """Sampler::sample on the current logits (modified in place)."""
        arr, n = _u32_array(recent)
        t = C.c_uint32()
        abi.check(_lib().aotk_sample(self.h, sampler.h, arr, n, C.byref(t)))
        return t.value

    def generate_sampled(self, sampler, pos, n, recent):
        """The app.rs:553-610 loop with `sampler`; `recent` = the tokens so far."""
        arr, nr = _u32_array(recent)
        out = (C.c_uint32 * n)()
        abi.check(_lib().aotk_generate(self.h, sampler.h, int(pos), int(n), arr, nr, out))
        return list(out)

    def save_prefix(self, tokens, n_cached):
        """prefix::serialize (prefix.rs:114-141): the AOTP v2 blob of `tokens`
        with the KV rows of their first n_cached positions."""
        arr = (C.c_uint32 * max(1, len(tokens)))(*[int(t) for t in tokens])
        n = C.c_size_t()
        abi.check(_lib().aotk_prefix_save(self.h, arr, len(tokens), int(n_cached), None, 0, C.byref(n)))
        out = np.empty(n.value, np.uint8)
        abi.check(_lib().aotk_prefix_save(self.h, arr, len(tokens), int(n_cached), out.ctypes.data_as(C.c_void_p),
                                          out.size, C.byref(n)))
        return out.tobytes()

    def load_prefix(self, blob):
        """Prefix::parse + load_into (prefix.rs:48-108): returns (tokens, n_cached)."""
        blob = bytes(blob)
        buf = np.frombuffer(blob, np.uint8)
        n, nc = C.c_size_t(), C.c_size_t()
        ptr = buf.ctypes.data_as(C.c_void_p) if buf.size else None
        abi.check(_lib().aotk_prefix_load(self.h, ptr, buf.size, None, 0, C.byref(n), C.byref(nc)))
        toks = (C.c_uint32 * n.value)()
        abi.check(_lib().aotk_prefix_load(self.h, ptr, buf.size, toks, n.value, C.byref(n), C.byref(nc)))
        return list(toks), nc.value

    def free(self):
        if self.h:
            _lib().aotk_state_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
