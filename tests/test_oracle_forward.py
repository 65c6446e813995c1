"""CPU tests: the oracle's model forward pinned against an independent f32
reference forward, as the reference pins its own compiled models.

crates/aot-llm/tests/e2e.rs builds tiny random models of every architecture
(`build_model`, :406-437), runs the compiled binary at batch 1 and batch 128
and compares its logits with `reference_logits` (:260-343): a plain f32
forward over the dequantized weights whose activations go through the same
int8 quantizers as the runtime (`act_quant`, :160-189). Because quantization
is discontinuous, an activation within float noise of a rounding boundary may
land on the other level; `check_quant_logits` (:504-537) allows up to two
such near-tie activations to be flipped, then holds the logits to
2e-3 * max|logit| + 1e-3 (:488-502) with the same argmax.

This file restates that reference forward in numpy, written from e2e.rs and
independent of oracle/oracle.c's forward, and checks the oracle's
forward / forward_batch against it for each architecture: llama, qwen2 (q/k/v
bias, NEOX), qwen3 (per-head q/k norms, head_dim 128 so q_dim > dim), phi3
(fused attn_qkv / ffn_up read through the GGUF model table), gemma3 (embedding
scale, post-norms, GeGLU, 5 sliding-window layers of window 4 with their own
RoPE base and one global layer with linear RoPE scaling), plus the three
benchmark quantization mixes at tiny shapes. The only oracle functions the
restatement uses are the dequantizers and the Q8_0 / Q8_K activation
quantizers, which tests/test_oracle.py pins against quant.rs's own vectors.
A mistake in the oracle's operator order (a post-norm in the wrong place, a
wrong RoPE base or layout, a missing bias or scale, a wrong window) moves the
logits by far more than the tolerance.
"""
import itertools

import numpy as np
import pytest

from oracle import oracle as O
from e2e_models import Rng, build_e2e_blob

TIE = 1e-5  # e2e.rs:33
F32_KIND = 0
Q8_0_KINDS = (3, 4, 5)
Q8_K_KINDS = (6, 7, 8)
f32 = np.float32

CASES = ["tiny-llama", "tiny-qwen2", "tiny-qwen3", "tiny-phi3", "tiny-gemma3", "tiny-q4km", "tiny-q8_0", "tiny-q5km"]


def test_e2e_rng_stream():
    """The generator is e2e.rs:81-95 step for step (a pure-Python loop)."""
    s = 0x5EED
    want = []
    M = 0xFFFFFFFFFFFFFFFF
    for _ in range(200):
        s ^= (s << 13) & M
        s ^= s >> 7
        s ^= (s << 17) & M
        want.append(f32(f32(f32(s % 1000001) / f32(500000.0) - f32(1.0)) * f32(0.2)))
    r = Rng(0x5EED)
    got = np.concatenate([r.vec(150, 0.2), r.vec(50, 0.2)])
    assert np.array_equal(got, np.array(want, np.float32))


# ------------------------------------------------------ reference forward

class Acts:
    """e2e.rs:139-156: activation quantization on, the near-ties seen, and
    the one to round the other way."""

    def __init__(self, flip=None):
        self.ties = []
        self.flip = flip


def act_quant(kind, x, acts):
    """e2e.rs:160-189."""
    if kind in Q8_0_KINDS:
        b = O.quantize_q8_0(x)
        q, d = b["qs"].ravel().astype(np.int32), np.repeat(b["d"], 32)
    elif kind in Q8_K_KINDS:
        b = O.quantize_q8_k(x)
        q, d = b["qs"].ravel().astype(np.int32), np.repeat(b["d"], 256)
    else:
        return x.copy()
    k_format = kind in Q8_K_KINDS
    with np.errstate(divide="ignore", invalid="ignore"):
        t = (x / d).astype(np.float32)
        near = (d != 0) & (np.abs(t - np.floor(t) - f32(0.5)) < f32(TIE) * np.maximum(np.abs(t), f32(1.0)))
    bits = x.view(np.uint32)
    for i in np.nonzero(near)[0]:
        key = (k_format, int(i), int(bits[i]))
        if key not in acts.ties:
            acts.ties.append(key)
    if acts.flip is not None and acts.flip[0] == k_format:
        i = acts.flip[1]
        if i < x.size and int(bits[i]) == acts.flip[2]:
            q = q.copy()
            q[i] = min(127, max(-127, q[i] + 1 if t[i] > q[i] else q[i] - 1))
    return (q.astype(np.float32) * d).astype(np.float32)


class RefModel:
    """The dequantized weights and hyper-parameters `reference_logits` reads."""

    def __init__(self, spec, blob):
        from aotk import abi
        s = spec.spec
        self.d = spec.d
        self.dims = s.dims
        self.flags = s.flags

        def w(t):
            if t.kind == abi.NONE:
                return None
            raw = blob[t.off:t.off + t.len]
            if t.rows == 1 and t.kind == F32_KIND:
                return raw.view("<f4").astype(np.float32)
            return (t.kind, O.dequant_rows(t.kind, raw, t.cols))

        self.embd = w(s.token_embd)
        self.output_norm = w(s.output_norm)
        self.output = w(s.output) if s.output.kind != abi.NONE else self.embd
        self.layers = []
        for li in range(spec.d["n_layer"]):
            L = spec.layers[li]
            self.layers.append({n: w(getattr(L, n)) for n in abi.LAYER_SLOTS if isinstance(getattr(L, n), abi.Tensor)}
                               | {"local": bool(L.local_attn)})


def matvec(m, x, acts):
    """e2e.rs:191-195 (f32 sums; the order is free, the tolerance covers it)."""
    kind, W = m
    xq = act_quant(kind, x, acts)
    return (W @ xq).astype(np.float32)


def rmsnorm(x, w, eps):
    """e2e.rs:197-201."""
    ss = f32(np.sum(x * x, dtype=np.float32) / f32(x.size))
    r = f32(1.0) / np.sqrt(f32(ss + f32(eps)))
    return (x * r * w).astype(np.float32)


def rope(x, n_heads, hd, pos, neox, base, scale):
    """e2e.rs:204-218 (rotary over the whole head)."""
    half = hd // 2
    i = np.arange(half, dtype=np.float32)
    theta = (f32(pos) / f32(scale)) * np.power(f32(base), -(f32(2.0) * i) / f32(hd), dtype=np.float32)
    c, s = np.cos(theta).astype(np.float32), np.sin(theta).astype(np.float32)
    x = x.reshape(n_heads, hd).copy()
    i0 = np.arange(half) if neox else 2 * np.arange(half)
    i1 = i0 + half if neox else i0 + 1
    a, b = x[:, i0].copy(), x[:, i1].copy()
    x[:, i0] = a * c - b * s
    x[:, i1] = a * s + b * c
    return x.ravel()


def norm_heads(x, w, n_heads, hd, eps):
    """e2e.rs:226-231."""
    return np.concatenate([rmsnorm(x[h * hd:(h + 1) * hd], w, eps) for h in range(n_heads)])


def reference_logits(m, tokens, acts):
    """e2e.rs:260-343: logits of the last token."""
    d, dims, fl = m.d, m.dims, m.flags
    dim, hd, nh, nkv = d["dim"], d["head_dim"], d["n_head"], d["n_kv_head"]
    eps = f32(dims.eps)
    kv_dim = nkv * hd
    gqa = nh // nkv
    k_cache = [np.zeros((len(tokens), kv_dim), np.float32) for _ in m.layers]
    v_cache = [np.zeros((len(tokens), kv_dim), np.float32) for _ in m.layers]
    window = int(dims.swa_window)
    logits = None
    for pos, tok in enumerate(tokens):
        x = m.embd[1][tok].copy()
        if fl.embd_scale:
            x = (x * np.sqrt(f32(dim))).astype(np.float32)
        for li, L in enumerate(m.layers):
            local = L["local"]
            base, scale = (dims.rope_base_local, dims.rope_scale_local) if local else (dims.rope_base, dims.rope_scale)
            t_start = pos + 1 - window if local and pos + 1 > window else 0
            xb = rmsnorm(x, L["attn_norm"], eps)
            q = matvec(L["wq"], xb, acts)
            k = matvec(L["wk"], xb, acts)
            v = matvec(L["wv"], xb, acts)
            if L["bq"] is not None:
                q, k, v = q + L["bq"], k + L["bk"], v + L["bv"]
            if L["q_norm"] is not None:
                q = norm_heads(q, L["q_norm"], nh, hd, eps)
                k = norm_heads(k, L["k_norm"], nkv, hd, eps)
            q = rope(q, nh, hd, pos, fl.rope_neox, base, scale)
            k = rope(k, nkv, hd, pos, fl.rope_neox, base, scale)
            k_cache[li][pos], v_cache[li][pos] = k, v
            att = np.zeros(nh * hd, np.float32)
            for h in range(nh):
                kvh = h // gqa
                qh = q[h * hd:(h + 1) * hd]
                kt = k_cache[li][t_start:pos + 1, kvh * hd:(kvh + 1) * hd]
                sc = (kt @ qh).astype(np.float32) / np.sqrt(f32(hd))
                e = np.exp(sc - sc.max()).astype(np.float32)
                p = (e / np.sum(e, dtype=np.float32)).astype(np.float32)
                att[h * hd:(h + 1) * hd] = p @ v_cache[li][t_start:pos + 1, kvh * hd:(kvh + 1) * hd]
            o = matvec(L["wo"], att, acts)
            if L["attn_post_norm"] is not None:
                o = rmsnorm(o, L["attn_post_norm"], eps)
            x = (x + o).astype(np.float32)
            xb = rmsnorm(x, L["ffn_norm"], eps)
            g = matvec(L["gate"], xb, acts)
            u = matvec(L["up"], xb, acts)
            if fl.gelu:
                hbuf = f32(0.5) * g * (f32(1.0) + np.tanh(f32(0.7978846) * (g + f32(0.044715) * g * g * g))) * u
            else:
                hbuf = g / (f32(1.0) + np.exp(-g)) * u
            dn = matvec(L["down"], hbuf.astype(np.float32), acts)
            if L["ffn_post_norm"] is not None:
                dn = rmsnorm(dn, L["ffn_post_norm"], eps)
            x = (x + dn).astype(np.float32)
        if pos + 1 == len(tokens):
            xb = rmsnorm(x, m.output_norm, eps)
            logits = matvec(m.output, xb, acts)
    return logits


def quant_reference(m, tokens):
    """e2e.rs:474-479: the logits and the change each near-tie flip makes."""
    acts = Acts()
    logits = reference_logits(m, tokens, acts)
    flips = [reference_logits(m, tokens, Acts(flip=t)) - logits for t in acts.ties]
    return logits, flips


def tolerance(expected):
    """e2e.rs:500-502."""
    return f32(2e-3) * np.abs(expected).max() + f32(1e-3)


def check_quant_logits(label, got, ref):
    """e2e.rs:504-537: the fewest (at most two) near-tie flips that explain
    the logits, then the usual tolerance and the same argmax."""
    logits, flips = ref
    n = len(flips)
    combos = itertools.chain([()], ((i,) for i in range(n)), itertools.combinations(range(n), 2))
    chosen = ()
    for c in combos:
        e = logits + sum((flips[i] for i in c), np.zeros_like(logits))
        if np.all(np.abs(got - e) <= tolerance(e)):
            chosen = c
            break
    expected = logits + sum((flips[i] for i in chosen), np.zeros_like(logits))
    err = float(np.abs(got - expected).max())
    assert err <= tolerance(expected), f"{label}: max error {err} (range {np.abs(expected).max()}, {n} near-ties)"
    # e2e.rs:488: max_by(total_cmp) -> the last of equal maxima; the data has no ties at the max.
    assert int(np.argmax(got)) == int(np.argmax(expected)), f"{label}: argmax differs"
    return chosen, n


def _model(name):
    from aotk import configs
    spec = configs.build(name)
    blob = build_e2e_blob(spec)
    n = 13 if spec.spec.dims.swa_window else 7  # e2e.rs:561-564: Gemma's prompt is longer than the window
    toks = configs.prompt_tokens(0xE2E, n, spec.d["vocab"])
    return spec, blob, toks


def _oracle_logits(spec, blob, toks, batch):
    m = O.Model(spec, blob, ctx=len(toks) + 1, max_batch=64, n_threads=4)
    if batch == 1:
        for i, t in enumerate(toks):
            m.forward(t, i, i + 1 == len(toks))
    else:
        m.prompt(toks, batch=batch)
    out = m.logits()
    m.close()
    return out


@pytest.mark.parametrize("name", CASES)
def test_oracle_forward_matches_reference_logits(name):
    """e2e.rs:565-575: batch 1 and batched prompt (the reference's 128; here
    64, the whole prompt in one chunk) against reference_logits."""
    spec, blob, toks = _model(name)
    run_spec, run_blob = spec, blob
    if name == "tiny-phi3":
        # the oracle reads Phi-3's fused tensors through the GGUF model table
        from aotk import gguf
        b = gguf.config_gguf(spec, blob, "phi3", fuse=True)
        f = gguf.GgufFile(b)
        run_spec = gguf.GgufSpec(f)
        run_blob = np.frombuffer(b, np.uint8)[f.data_offset:f.data_offset + f.data_len()].copy()
        assert run_spec.layers[0].wk.off == run_spec.layers[0].wq.off + run_spec.layers[0].wq.len
    ref = quant_reference(RefModel(spec, blob), toks)
    assert np.abs(ref[0]).max() > 1.0, "degenerate logits would make the tolerance meaningless"
    one = _oracle_logits(run_spec, run_blob, toks, 1)
    many = _oracle_logits(run_spec, run_blob, toks, 64)
    check_quant_logits(f"{name} batch 1", one, ref)
    check_quant_logits(f"{name} batch 64", many, ref)
    assert np.array_equal(one.view(np.uint32), many.view(np.uint32)), "batched forward != token by token"


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-gemma3"])
def test_reference_logits_catch_operator_mistakes(name, monkeypatch):
    """The pin has teeth: each of these plausible mistakes, made in the
    restatement, moves the logits beyond the tolerance."""
    spec, blob, toks = _model(name)
    m = RefModel(spec, blob)
    good = reference_logits(m, toks, Acts())
    mistakes = []
    # a wrong RoPE layout
    m.flags.rope_neox ^= 1
    mistakes.append(reference_logits(m, toks, Acts()))
    m.flags.rope_neox ^= 1
    # a wrong RoPE base
    old = m.dims.rope_base
    m.dims.rope_base = old * 2
    mistakes.append(reference_logits(m, toks, Acts()))
    m.dims.rope_base = old
    if name == "tiny-gemma3":
        # the global base on the local layers
        old = m.dims.rope_base_local
        m.dims.rope_base_local = m.dims.rope_base
        mistakes.append(reference_logits(m, toks, Acts()))
        m.dims.rope_base_local = old
        # the sliding window ignored
        w = m.dims.swa_window
        m.dims.swa_window = 1 << 20
        mistakes.append(reference_logits(m, toks, Acts()))
        m.dims.swa_window = w
        # no embedding scale
        m.flags.embd_scale = 0
        mistakes.append(reference_logits(m, toks, Acts()))
        m.flags.embd_scale = 1
        # post-norms left out
        saved = [(L["attn_post_norm"], L["ffn_post_norm"]) for L in m.layers]
        for L in m.layers:
            L["attn_post_norm"] = L["ffn_post_norm"] = None
        mistakes.append(reference_logits(m, toks, Acts()))
        for L, (a, b) in zip(m.layers, saved):
            L["attn_post_norm"], L["ffn_post_norm"] = a, b
    for i, bad in enumerate(mistakes):
        assert np.abs(bad - good).max() > 1.5 * tolerance(good), f"mistake {i} not detected"
