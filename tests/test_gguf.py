"""GGUF ingestion (crates/aot-gguf/src/lib.rs, crates/aot-codegen/src/model.rs).

CPU: the reference's own parser tests (lib.rs:513-552) on aotk.gguf, the
parser's error paths, and the model table read back from files written for
every test architecture (dims, flags and tensor table equal to the config's,
data section equal to the blob; Phi-3's fused q/k/v and gate/up as row
views). GPU: models loaded from GGUF files give the logits of the same model
built from the config, and a fused Phi-3 file runs bit-exact with the oracle."""
import struct

import numpy as np
import pytest

TINY = ["tiny-llama", "tiny-qwen2", "tiny-qwen3", "tiny-gemma3", "tiny-q4km", "tiny-q8_0", "tiny-q5km"]


def _g():
    from aotk import gguf
    return gguf


def test_reference_roundtrip():
    gg = _g()
    w = gg.GgufWriter()
    w.kv("general.architecture", gg.Meta(gg.STRING, "llama"))
    w.kv("llama.block_count", gg.Meta(gg.U32, 2))
    w.kv("tokenizer.ggml.tokens", gg.Meta(gg.ARRAY, [gg.Meta(gg.STRING, "a"), gg.Meta(gg.STRING, "b")]))
    w.tensor("x", [4, 2], 0, bytes(32))
    w.tensor("y", [32], 2, bytes([1]) * 18)
    b = w.finish()
    f = gg.GgufFile(b, len(b))
    assert f.version == 3
    assert f.architecture() == "llama"
    assert f.get_u64("llama.block_count") == 2
    assert len(f.get_array("tokenizer.ggml.tokens")) == 2
    assert len(f.tensors) == 2
    x = f.tensor("x")
    assert x.rows() == 2 and x.cols() == 4 and x.n_bytes() == 32
    y = f.tensor("y")
    assert y.offset == 32
    assert f.data_offset % 32 == 0
    assert b[f.data_offset + 32:f.data_offset + 50] == bytes([1]) * 18


def test_reference_rejects():
    gg = _g()
    with pytest.raises(gg.GgufError, match="bad magic"):
        gg.GgufFile(bytes(32), 32)
    w = gg.GgufWriter()
    w.kv("k", gg.Meta(gg.U32, 1))
    b = w.finish()
    with pytest.raises(gg.GgufError, match="truncated"):
        gg.GgufFile(b[:12], 12)


def test_parser_errors():
    gg = _g()

    def file(version=3, kvs=(), tensors=()):
        out = bytearray(struct.pack("<IIQQ", gg.GGUF_MAGIC, version, len(tensors), len(kvs)))
        for k, raw in kvs:
            out += struct.pack("<Q", len(k)) + k.encode() + raw
        for name, dims, ty, off in tensors:
            out += struct.pack("<Q", len(name)) + name.encode() + struct.pack("<I", len(dims))
            out += b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", ty, off)
        out += bytes((-len(out)) % 32) + bytes(64)
        return bytes(out)

    with pytest.raises(gg.GgufError, match="version"):
        gg.GgufFile(file(version=4))
    with pytest.raises(gg.GgufError, match="alignment"):
        gg.GgufFile(file(kvs=[("general.alignment", struct.pack("<II", gg.U32, 48))]))
    with pytest.raises(gg.GgufError, match="value type"):
        gg.GgufFile(file(kvs=[("k", struct.pack("<I", 13))]))
    with pytest.raises(gg.GgufError, match="UTF-8"):
        gg.GgufFile(file(kvs=[("k", struct.pack("<IQ", gg.STRING, 2) + b"\xff\xfe")]))
    with pytest.raises(gg.GgufError, match="dimensions"):
        gg.GgufFile(file(tensors=[("t", [1, 1, 1, 1, 1], 0, 0)]))
    with pytest.raises(gg.GgufError, match="tensor type"):
        gg.GgufFile(file(tensors=[("t", [4], 5, 0)]))
    with pytest.raises(gg.GgufError, match="exceeds file size"):
        gg.GgufFile(file(tensors=[("t", [64], 0, 32)]))
    # an alignment of 64 moves the data section
    f = gg.GgufFile(file(kvs=[("general.alignment", struct.pack("<II", gg.U32, 64))], tensors=[("t", [4], 0, 0)]))
    assert f.alignment == 64 and f.data_offset % 64 == 0


def _config_file(oracle, name, arch=None, fuse=False):
    from aotk import configs
    gg = _g()
    spec = configs.build(name)
    blob = oracle.synth_blob(spec, 0x5EED)
    b = gg.config_gguf(spec, blob, arch or spec.cfg["arch"], fuse=fuse)
    return spec, blob, b


def _tensors(spec):
    s = spec.spec
    out = [("token_embd", s.token_embd), ("output_norm", s.output_norm), ("output", s.output), ("rope_freqs", s.rope_freqs)]
    from aotk import abi
    for li in range(spec.d["n_layer"]):
        L = spec.layers[li]
        out += [(f"{li}.{n}", getattr(L, n)) for n in abi.LAYER_SLOTS]
        out.append((f"{li}.local", L.local_attn))
    return out


def _fields(t):
    return t if isinstance(t, int) else (t.kind, t.off, t.len, t.rows, t.cols) if t.kind >= 0 else (t.kind,)


@pytest.mark.parametrize("name", TINY)
def test_model_table_matches_config(oracle, name):
    gg = _g()
    spec, blob, b = _config_file(oracle, name)
    f = gg.GgufFile(b)
    gs = gg.GgufSpec(f)
    assert gs.warnings == []
    for k in ("dim", "hidden", "n_layer", "n_head", "n_kv_head", "head_dim", "rot_dim", "vocab", "n_ctx_train", "swa_window"):
        assert getattr(gs.spec.dims, k) == getattr(spec.spec.dims, k), k
    for k in ("eps", "rope_base", "rope_scale", "rope_base_local", "rope_scale_local"):
        assert np.float32(getattr(gs.spec.dims, k)) == np.float32(getattr(spec.spec.dims, k)), k
    for k in ("rope_neox", "qkv_bias", "qk_norm", "embd_scale", "post_norms", "gelu", "swa_pattern"):
        assert getattr(gs.spec.flags, k) == getattr(spec.spec.flags, k), k
    for (n1, t1), (n2, t2) in zip(_tensors(spec), _tensors(gs)):
        assert _fields(t1) == _fields(t2), n1
    assert bytes(b[f.data_offset:f.data_offset + f.data_len()]) == bytes(blob[:f.data_len()])


def test_phi3_fused_views(oracle):
    gg = _g()
    spec, blob, b = _config_file(oracle, "tiny-q8_0", arch="phi3", fuse=True)
    f = gg.GgufFile(b)
    gs = gg.GgufSpec(f)
    assert gs.spec.flags.rope_neox == 1
    data = b[f.data_offset:]
    for li in range(spec.d["n_layer"]):
        A, B = spec.layers[li], gs.layers[li]
        qkv = f.tensor(f"blk.{li}.attn_qkv.weight")
        assert B.wq.off == qkv.offset and B.wk.off == B.wq.off + B.wq.len and B.wv.off == B.wk.off + B.wk.len
        for slot in ("wq", "wk", "wv", "gate", "up"):
            x, y = getattr(A, slot), getattr(B, slot)
            assert (x.rows, x.cols, x.len) == (y.rows, y.cols, y.len)
            assert data[y.off:y.off + y.len] == bytes(blob[x.off:x.off + x.len]), (li, slot)


def test_model_table_errors(oracle):
    gg = _g()
    _, _, good = _config_file(oracle, "tiny-llama")
    gg.GgufSpec(gg.GgufFile(good))

    def rewrite(edit_kv=None, edit_t=None, drop_key=None):
        f = gg.GgufFile(good)
        w = gg.GgufWriter()
        for k, v in f.metadata:
            if k == drop_key:
                continue
            w.kv(k, edit_kv(k, v) if edit_kv else v)
        data = good[f.data_offset:]
        ts = [(t.name, t.dims, t.ty, data[t.offset:t.offset + t.n_bytes()]) for t in f.tensors]
        if edit_t:
            ts = edit_t(ts)
        for t in ts:
            w.tensor(*t)
        return gg.GgufFile(w.finish())

    arch = lambda a: (lambda k, v: gg.Meta(gg.STRING, a) if k == "general.architecture" else v)  # noqa: E731
    with pytest.raises(gg.GgufError, match="unsupported architecture"):
        gg.GgufSpec(rewrite(arch("mamba")))
    with pytest.raises(gg.GgufError, match="not found"):
        gg.GgufSpec(rewrite(drop_key="llama.block_count"))
    with pytest.raises(gg.GgufError, match="bias tensors are not supported"):
        gg.GgufSpec(rewrite(edit_t=lambda ts: ts + [("blk.0.attn_q.bias", [256], 0, bytes(1024))]))
    with pytest.raises(gg.GgufError, match="expected shape"):
        gg.GgufSpec(rewrite(edit_t=lambda ts: [(n, d[::-1] if n == "blk.0.attn_k.weight" else d, t, x) for n, d, t, x in ts]))
    with pytest.raises(gg.GgufError, match="must be f32"):
        gg.GgufSpec(rewrite(edit_t=lambda ts: [(n, d, 1 if n == "output_norm.weight" else t, x[:len(x) // 2] if n == "output_norm.weight" else x)
                                               for n, d, t, x in ts]))
    with pytest.raises(gg.GgufError, match="LongRoPE"):
        gg.GgufSpec(rewrite(edit_t=lambda ts: ts + [("rope_factors_long.weight", [32], 0, bytes(128))]))
    # an unused tensor other than a bias is ignored with a warning
    gs = gg.GgufSpec(rewrite(edit_t=lambda ts: ts + [("extra.weight", [32], 0, bytes(128))]))
    assert gs.warnings and "extra.weight" in gs.warnings[0]
    _, _, gem = _config_file(oracle, "tiny-gemma3")
    f = gg.GgufFile(gem)
    w = gg.GgufWriter()
    for k, v in f.metadata:
        if k != "gemma3.attention.sliding_window":
            w.kv(k, v)
    for t in f.tensors:
        w.tensor(t.name, t.dims, t.ty, gem[f.data_offset + t.offset:f.data_offset + t.offset + t.n_bytes()])
    with pytest.raises(gg.GgufError, match="sliding_window"):
        gg.GgufSpec(gg.GgufFile(w.finish()))


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["tiny-llama", "tiny-gemma3", "tiny-q5km"])
def test_load_gguf_file(aotk, oracle, name, tmp_path):
    from aotk import configs, gguf
    spec, blob, b = _config_file(oracle, name)
    path = tmp_path / "m.gguf"
    path.write_bytes(b)
    gs, data = gguf.open_model(str(path))
    toks = configs.prompt_tokens(4, 9, spec.d["vocab"])
    a = aotk.State(aotk.Model(gs, np.frombuffer(data, np.uint8)), 32)
    c = aotk.State(aotk.Model(spec, blob), 32)
    a.prompt(toks)
    c.prompt(toks)
    assert np.array_equal(a.logits(), c.logits())
    assert a.generate(len(toks), 6) == c.generate(len(toks), 6)


@pytest.mark.gpu
def test_phi3_fused_model(aotk, oracle, tmp_path):
    from aotk import configs, gguf
    spec, blob, b = _config_file(oracle, "tiny-q8_0", arch="phi3", fuse=True)
    path = tmp_path / "phi3.gguf"
    path.write_bytes(b)
    gs, data = gguf.open_model(str(path))
    data = np.frombuffer(data, np.uint8).copy()
    toks = configs.prompt_tokens(8, 11, spec.d["vocab"])
    ref = oracle.Model(gs, data, 32)
    st = aotk.State(aotk.Model(gs, data), 32)
    ref.prompt(toks)
    st.prompt(toks)
    assert np.array_equal(st.logits(), ref.logits())
    assert st.generate(len(toks), 8) == ref.generate(len(toks), 8)
