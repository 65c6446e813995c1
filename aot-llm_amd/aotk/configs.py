"""Model graphs of the five benchmark configurations and the small test models.

A config becomes an `aotk_model_spec` (the tensor table aot-codegen bakes into
the generated model.rs: crates/aot-codegen/src/emit.rs:399-464) laid out like
a GGUF tensor-data section (tensors 32-byte aligned, aot-gguf/src/lib.rs:23).
Architecture switches follow crates/aot-codegen/src/model.rs:183-192; Gemma 3
local layers are every layer with (i + 1) % 6 != 0 (model.rs:351).
"""
import ctypes as C

from . import abi

ALIGN = 32

# Quantization mixes named in the benchmark configurations.
#   q4_k_m: Q4_K {q, k, o, gate, up, embd}, Q6_K {v, down, output}
#   q5_k_m: Q5_K {q, k, o, gate, up},        Q6_K {v, down, output/embd}
#   q8_0:   every matrix Q8_0
MIXES = {
    "q4_k_m": dict(wq=abi.Q4_K, wk=abi.Q4_K, wv=abi.Q6_K, wo=abi.Q4_K, gate=abi.Q4_K, up=abi.Q4_K,
                   down=abi.Q6_K, embd=abi.Q4_K, output=abi.Q6_K),
    "q5_k_m": dict(wq=abi.Q5_K, wk=abi.Q5_K, wv=abi.Q6_K, wo=abi.Q5_K, gate=abi.Q5_K, up=abi.Q5_K,
                   down=abi.Q6_K, embd=abi.Q6_K, output=abi.Q6_K),
    "q8_0": dict(wq=abi.Q8_0, wk=abi.Q8_0, wv=abi.Q8_0, wo=abi.Q8_0, gate=abi.Q8_0, up=abi.Q8_0,
                 down=abi.Q8_0, embd=abi.Q8_0, output=abi.Q8_0),
}

ARCH_FLAGS = {
    # model.rs:183-192
    "llama": dict(),
    "qwen2": dict(rope_neox=1, qkv_bias=1),
    "qwen3": dict(rope_neox=1, qk_norm=1),
    "gemma3": dict(rope_neox=1, qk_norm=1, embd_scale=1, post_norms=1, gelu=1, swa_pattern=6),
    # Phi-3: NEOX RoPE; its fused attn_qkv / ffn_up are row views of one
    # tensor (model.rs:257-262), the same arithmetic as separate tensors.
    "phi3": dict(rope_neox=1),
}

CONFIGS = {
    # TinyLlama-1.1B shape, Q4_K_M, 6-token prompt + 32 greedy
    "tinyllama-1.1b-q4km": dict(arch="llama", dim=2048, hidden=5632, n_layer=22, n_head=32, n_kv_head=4,
                                head_dim=64, vocab=32000, rope_base=10000.0, eps=1e-5, mix="q4_k_m",
                                n_ctx_train=2048),
    # Llama-3-8B shape, Q4_K_M, 512-token prompt in 64-chunks + 128 greedy
    "llama3-8b-q4km": dict(arch="llama", dim=4096, hidden=14336, n_layer=32, n_head=32, n_kv_head=8,
                           head_dim=128, vocab=128256, rope_base=500000.0, eps=1e-5, mix="q4_k_m",
                           n_ctx_train=8192),
    # Qwen3-8B shape, Q8_0, KV prefilled to 4096 + 256 greedy
    "qwen3-8b-q8_0": dict(arch="qwen3", dim=4096, hidden=12288, n_layer=36, n_head=32, n_kv_head=8,
                          head_dim=128, vocab=151936, rope_base=1000000.0, eps=1e-6, mix="q8_0",
                          n_ctx_train=40960),
    # Gemma-3-4B shape, Q5_K_M, 8192 context + 256 greedy (tied output)
    "gemma3-4b-q5km": dict(arch="gemma3", dim=2560, hidden=10240, n_layer=34, n_head=8, n_kv_head=4,
                           head_dim=256, vocab=262144, rope_base=1000000.0, eps=1e-6, mix="q5_k_m",
                           swa_window=1024, tied=True, n_ctx_train=131072),
}

# Small models in the spirit of the reference's e2e test (tests/e2e.rs:25-79,
# :433-434): layer 0 exercises the K-quants, layer 1 the float / Q8_0 / Q4_0
# kernels; kinds are listed as (wq, wk, wv, wo, gate, up, down).
E2E_KINDS = [
    (abi.Q4_K, abi.Q4_0, abi.Q8_0, abi.Q5_K, abi.Q4_K, abi.Q4_K, abi.Q6_K),
    (abi.F16, abi.BF16, abi.F32, abi.Q4_0, abi.Q8_0, abi.Q8_0, abi.Q5_0),
]
# Fused tensors share one format across their parts (tests/e2e.rs:416-421).
E2E_FUSED_KINDS = [tuple(k[i] for i in (0, 0, 0, 3, 4, 4, 6)) for k in E2E_KINDS]
TINY = dict(dim=256, hidden=512, n_head=4, n_kv_head=2, head_dim=64, vocab=512, eps=1e-5,
            rope_base=10000.0, n_ctx_train=512)
TEST_CONFIGS = {
    "tiny-llama": dict(TINY, arch="llama", n_layer=2, mix="e2e"),
    "tiny-qwen2": dict(TINY, arch="qwen2", n_layer=2, mix="e2e"),
    "tiny-qwen3": dict(TINY, arch="qwen3", n_layer=2, head_dim=128, mix="e2e"),
    "tiny-gemma3": dict(TINY, arch="gemma3", n_layer=6, mix="e2e", swa_window=4, rope_base=1000000.0,
                        rope_scale=2.0, tied=False),
    "tiny-phi3": dict(TINY, arch="phi3", n_layer=2, mix="e2e-fused"),
    "tiny-q4km": dict(TINY, arch="llama", n_layer=2, mix="q4_k_m"),
    "tiny-q8_0": dict(TINY, arch="qwen3", n_layer=2, head_dim=128, mix="q8_0"),
    "tiny-q5km": dict(TINY, arch="gemma3", n_layer=6, mix="q5_k_m", swa_window=4, tied=True),
}


def get(name):
    if name in CONFIGS:
        return dict(CONFIGS[name])
    return dict(TEST_CONFIGS[name])


class Spec:
    """A built spec: the ctypes struct (kept alive with its layer array), the
    blob length and the per-tensor table for reporting."""

    def __init__(self, cfg):
        self.cfg = cfg
        flags = ARCH_FLAGS[cfg["arch"]]
        d = dict(dim=cfg["dim"], hidden=cfg["hidden"], n_layer=cfg["n_layer"], n_head=cfg["n_head"],
                 n_kv_head=cfg["n_kv_head"], head_dim=cfg["head_dim"], vocab=cfg["vocab"])
        d["rot_dim"] = cfg.get("rot_dim", d["head_dim"])
        self.d = d
        q_dim = d["n_head"] * d["head_dim"]
        kv_dim = d["n_kv_head"] * d["head_dim"]
        self.off = 0
        self.tensors = []
        mix = cfg["mix"]

        def kind_of(slot, layer):
            if mix in ("e2e", "e2e-fused"):
                ks = (E2E_KINDS if mix == "e2e" else E2E_FUSED_KINDS)[layer % 2]
                idx = ("wq", "wk", "wv", "wo", "gate", "up", "down").index(slot)
                return ks[idx]
            return MIXES[mix][slot]

        embd_kind = abi.Q4_K if mix.startswith("e2e") else MIXES[mix]["embd"]
        out_kind = abi.Q6_K if mix.startswith("e2e") else MIXES[mix]["output"]
        self.spec = abi.ModelSpec()
        s = self.spec
        for k, v in d.items():
            setattr(s.dims, k, v)
        s.dims.n_ctx_train = cfg.get("n_ctx_train", 2048)
        s.dims.eps = cfg["eps"]
        s.dims.rope_base = cfg["rope_base"]
        s.dims.rope_scale = cfg.get("rope_scale", 1.0)
        s.dims.swa_window = cfg.get("swa_window", 0)
        s.dims.rope_base_local = 10000.0  # model.rs:350 (llama.cpp's Gemma 3 local base)
        s.dims.rope_scale_local = 1.0
        for k in ("rope_neox", "qkv_bias", "qk_norm", "embd_scale", "post_norms", "gelu"):
            setattr(s.flags, k, flags.get(k, 0))
        s.flags.swa_pattern = flags.get("swa_pattern", 0)
        s.token_embd = self._tensor("token_embd", embd_kind, d["vocab"], d["dim"])
        s.output_norm = self._tensor("output_norm", abi.F32, 1, d["dim"])
        if cfg.get("tied"):
            s.output = self._none()
        else:
            s.output = self._tensor("output", out_kind, d["vocab"], d["dim"])
        s.rope_freqs = self._none()
        self.layers = (abi.Layer * d["n_layer"])()
        for li in range(d["n_layer"]):
            L = self.layers[li]
            p = f"blk.{li}."
            L.attn_norm = self._tensor(p + "attn_norm", abi.F32, 1, d["dim"])
            L.wq = self._tensor(p + "attn_q", kind_of("wq", li), q_dim, d["dim"])
            L.wk = self._tensor(p + "attn_k", kind_of("wk", li), kv_dim, d["dim"])
            L.wv = self._tensor(p + "attn_v", kind_of("wv", li), kv_dim, d["dim"])
            L.wo = self._tensor(p + "attn_output", kind_of("wo", li), d["dim"], q_dim)
            L.ffn_norm = self._tensor(p + "ffn_norm", abi.F32, 1, d["dim"])
            L.gate = self._tensor(p + "ffn_gate", kind_of("gate", li), d["hidden"], d["dim"])
            L.up = self._tensor(p + "ffn_up", kind_of("up", li), d["hidden"], d["dim"])
            L.down = self._tensor(p + "ffn_down", kind_of("down", li), d["dim"], d["hidden"])
            if flags.get("qkv_bias"):
                L.bq = self._tensor(p + "attn_q.bias", abi.F32, 1, q_dim)
                L.bk = self._tensor(p + "attn_k.bias", abi.F32, 1, kv_dim)
                L.bv = self._tensor(p + "attn_v.bias", abi.F32, 1, kv_dim)
            else:
                L.bq = L.bk = L.bv = self._none()
            if flags.get("qk_norm"):
                L.q_norm = self._tensor(p + "attn_q_norm", abi.F32, 1, d["head_dim"])
                L.k_norm = self._tensor(p + "attn_k_norm", abi.F32, 1, d["head_dim"])
            else:
                L.q_norm = L.k_norm = self._none()
            if flags.get("post_norms"):
                L.attn_post_norm = self._tensor(p + "post_attention_norm", abi.F32, 1, d["dim"])
                L.ffn_post_norm = self._tensor(p + "post_ffw_norm", abi.F32, 1, d["dim"])
            else:
                L.attn_post_norm = L.ffn_post_norm = self._none()
            pat = flags.get("swa_pattern", 0)
            L.local_attn = 1 if (pat > 0 and (li + 1) % pat != 0) else 0
        s.layers = C.cast(self.layers, C.POINTER(abi.Layer))
        self.blob_len = (self.off + ALIGN - 1) // ALIGN * ALIGN

    def _none(self):
        t = abi.Tensor()
        t.kind = abi.NONE
        return t

    def _tensor(self, name, kind, rows, cols):
        t = abi.Tensor()
        t.kind = kind
        t.rows = rows
        t.cols = cols
        t.len = rows * abi.row_bytes(kind, cols)
        self.off = (self.off + ALIGN - 1) // ALIGN * ALIGN
        t.off = self.off
        self.off += t.len
        self.tensors.append((name, kind, rows, cols, t.off, t.len))
        return t

    def ptr(self):
        return C.pointer(self.spec)

    @property
    def out_tensor(self):
        return self.spec.output if self.spec.output.kind != abi.NONE else self.spec.token_embd

    def decode_weight_bytes(self):
        """Weight bytes one decode step streams: every layer matrix plus the
        lm-head and the embedding row (state.rs:199-245 views)."""
        total = 0
        for li in range(self.d["n_layer"]):
            L = self.layers[li]
            for slot in ("wq", "wk", "wv", "wo", "gate", "up", "down"):
                total += getattr(L, slot).len
        total += self.out_tensor.len
        total += abi.row_bytes(self.spec.token_embd.kind, self.d["dim"])
        return total


def build(name_or_cfg):
    cfg = get(name_or_cfg) if isinstance(name_or_cfg, str) else name_or_cfg
    return Spec(cfg)


def prompt_tokens(seed, n, vocab):
    """Uniform random token ids (splitmix64 stream of `seed`)."""
    out = []
    z = seed & 0xFFFFFFFFFFFFFFFF
    for _ in range(n):
        z = (z + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        x = z
        x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        x ^= x >> 31
        out.append(x % vocab)
    return out
