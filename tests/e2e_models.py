"""Tiny random models built like crates/aot-llm/tests/e2e.rs builds its own
(test helper, shared by the CPU pin of the oracle forward and the GPU model
tests)."""
import ctypes as C

import numpy as np

from oracle import oracle as O

f32 = np.float32


class Rng:
    """e2e.rs:81-95 (xorshift64 13/7/17, uniform in [-a, a])."""

    def __init__(self, seed):
        self.state = C.c_uint64(seed)

    def vec(self, n, a):
        out = np.empty(n, np.float32)
        O.load().or_e2e_uniform(C.byref(self.state), a, O.ptr(out), n)
        return out



def build_e2e_blob(spec, seed=0x5EED):
    """e2e.rs:406-437 `build_model`, in its generation order, written into the
    tensor layout of `spec`: matrices uniform(+-0.2) (down 0.14, embedding
    1.0) quantized row by row with the reference encoders, norms 1 + u(0.5),
    biases u(0.3)."""
    from aotk import abi
    blob = np.zeros(spec.blob_len, np.uint8)
    rng = Rng(seed)
    s = spec.spec

    def put(t, data):
        data = np.ascontiguousarray(data).view(np.uint8).ravel()
        assert data.size == t.len
        blob[t.off:t.off + t.len] = data

    def norm(t):
        put(t, (f32(1.0) + rng.vec(t.cols, 0.5)).astype("<f4"))

    def mat(t, amp):
        raw = rng.vec(t.rows * t.cols, amp).reshape(t.rows, t.cols)
        put(t, O.quantize_rows(t.kind, raw))

    for li in range(spec.d["n_layer"]):
        L = spec.layers[li]
        norm(L.attn_norm)
        for slot in ("wq", "wk", "wv", "wo"):
            mat(getattr(L, slot), 0.2)
        norm(L.ffn_norm)
        mat(L.gate, 0.2)
        mat(L.up, 0.2)
        mat(L.down, 0.14)
        for slot in ("bq", "bk", "bv"):
            t = getattr(L, slot)
            if t.kind != abi.NONE:
                put(t, rng.vec(t.cols, 0.3).astype("<f4"))
        for slot in ("q_norm", "k_norm", "attn_post_norm", "ffn_post_norm"):
            t = getattr(L, slot)
            if t.kind != abi.NONE:
                norm(t)
    mat(s.token_embd, 1.0)
    norm(s.output_norm)
    if s.output.kind != abi.NONE:
        mat(s.output, 0.2)
    return blob
