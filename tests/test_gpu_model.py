"""Whole-model parity: the HIP forward against the oracle's emitted forward."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TINY = ["tiny-llama", "tiny-qwen2", "tiny-qwen3", "tiny-gemma3", "tiny-q4km", "tiny-q8_0", "tiny-q5km"]


def rel_l2(a, b):
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("name", TINY)
def test_synthetic_weights_bitexact(aotk, oracle, name):
    from aotk import configs
    spec = configs.build(name)
    blob = oracle.synth_blob(spec, 0x5EED)
    m = aotk.Model(spec, seed=0x5EED)
    assert np.array_equal(m.download(), blob)


@pytest.mark.parametrize("name", TINY)
def test_forward_logits_and_greedy(aotk, oracle, name):
    from aotk import configs
    spec = configs.build(name)
    blob = oracle.synth_blob(spec, 0x5EED)
    ctx = 48
    ref = oracle.Model(spec, blob, ctx)
    gm = aotk.Model(spec, blob)
    st = aotk.State(gm, ctx)
    toks = configs.prompt_tokens(7, 9, spec.d["vocab"])
    ref.prompt(toks)
    st.prompt(toks)
    a, b = st.logits(), ref.logits()
    assert rel_l2(a, b) < 1e-3, rel_l2(a, b)
    assert np.array_equal(a, b), f"logits not bit-exact (rel L2 {rel_l2(a, b):.3g})"
    assert int(np.argmax(a)) == oracle.argmax(b)
    n = 16
    assert st.generate(len(toks), n) == ref.generate(len(toks), n)


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-gemma3"])
def test_batch_matches_single(aotk, oracle, name):
    from aotk import configs
    spec = configs.build(name)
    gm = aotk.Model(spec, seed=3)
    toks = configs.prompt_tokens(3, 12, spec.d["vocab"])
    s1, s2 = aotk.State(gm, 32), aotk.State(gm, 32)
    s1.prompt(toks, batch=64)
    for i, t in enumerate(toks):
        s2.forward(t, i, i + 1 == len(toks))
    assert np.array_equal(s1.logits(), s2.logits())


def test_errors(aotk):
    from aotk import configs
    spec = configs.build("tiny-llama")
    gm = aotk.Model(spec, seed=1)
    st = aotk.State(gm, 8, 4)
    with pytest.raises(aotk.AotkError, match="out of range"):
        st.forward(10 ** 6, 0)
    with pytest.raises(aotk.AotkError, match="exceeds the context"):
        st.forward(1, 8)
    with pytest.raises(aotk.AotkError, match="batch size"):
        st.forward_batch([1] * 5, 0)


def test_tinyllama_config_greedy_stream(aotk, oracle):
    """TinyLlama shape Q4_K_M, 6-token prompt, 32 greedy tokens."""
    from aotk import configs
    spec = configs.build("tinyllama-1.1b-q4km")
    gm = aotk.Model(spec, seed=0x5EED)
    blob = gm.download()
    toks = configs.prompt_tokens(1, 6, spec.d["vocab"])
    ctx = 38
    st = aotk.State(gm, ctx)
    st.prompt(toks)
    ref = oracle.Model(spec, blob, ctx)
    ref.prompt(toks)
    assert rel_l2(st.logits(), ref.logits()) < 1e-3
    assert np.array_equal(st.logits(), ref.logits())
    assert st.generate(6, 32) == ref.generate(6, 32)


E2E_CASES = ["tiny-llama", "tiny-qwen2", "tiny-qwen3", "tiny-phi3", "tiny-gemma3", "tiny-q4km", "tiny-q8_0", "tiny-q5km"]


@pytest.mark.parametrize("name", E2E_CASES)
def test_e2e_models_bitexact(aotk, oracle, name):
    """The models tests/test_oracle_forward.py pins the oracle's forward with
    (built like crates/aot-llm/tests/e2e.rs:406-437, larger weights than the
    synthetic generator), token by token and batched, on the GPU: logits bit
    for bit equal to the oracle's, and the same greedy continuation."""
    from aotk import configs, gguf
    from e2e_models import build_e2e_blob
    spec = configs.build(name)
    blob = build_e2e_blob(spec)
    if name == "tiny-phi3":
        b = gguf.config_gguf(spec, blob, "phi3", fuse=True)
        f = gguf.GgufFile(b)
        spec = gguf.GgufSpec(f)
        blob = np.frombuffer(b, np.uint8)[f.data_offset:f.data_offset + f.data_len()].copy()
    n = 13 if spec.spec.dims.swa_window else 7
    toks = configs.prompt_tokens(0xE2E, n, spec.d["vocab"])
    ctx = n + 10
    gm = aotk.Model(spec, blob)
    for batch in (1, 64):
        ref = oracle.Model(spec, blob, ctx)
        st = aotk.State(gm, ctx)
        if batch == 1:
            for i, t in enumerate(toks):
                ref.forward(t, i, i + 1 == n)
                st.forward(t, i, i + 1 == n)
        else:
            ref.prompt(toks, batch=batch)
            st.prompt(toks, batch=batch)
        a, b = st.logits(), ref.logits()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"batch {batch}: rel L2 {rel_l2(a, b):.3g}"
        assert st.generate(n, 8) == ref.generate(n, 8)
        ref.close()


@pytest.mark.parametrize("name", ["tiny-llama", "tiny-qwen3", "tiny-gemma3"])
@pytest.mark.parametrize("ctx", [320, 321])
def test_decode_attention_at_the_one_launch_bound(aotk, oracle, name, ctx):
    """Decode steps at positions ~310 of a state whose context is 320 (every
    layer's span fits the one-launch decode attention) and 321 (the global
    layers take the scores + softmax/output pair): streams and last logits
    equal the oracle's bit for bit (q/k norms in Qwen3, sliding-window local
    layers in Gemma-3)."""
    from aotk import configs
    spec = configs.build(name)
    blob = oracle.synth_blob(spec, 0x5EED)
    n = ctx - 10
    toks = configs.prompt_tokens(3, n, spec.d["vocab"])
    print(f"[decode1] {name} ctx {ctx}", flush=True)
    gm = aotk.Model(spec, blob)
    st = aotk.State(gm, ctx)
    ref = oracle.Model(spec, blob, ctx)
    try:
        st.prompt(toks, batch=64)
        ref.prompt(toks, batch=64)
        assert st.generate(n, 8) == ref.generate(n, 8)
        a, b = st.logits(), ref.logits()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"rel L2 {rel_l2(a, b):.3g}"
    finally:
        ref.close()
        st.free()
        gm.free()


def test_generate_fills_the_whole_context(aotk, oracle):
    """A generation of ctx + 1 tokens from position 0 (forwards at every
    position of the context) keeps all of its token history: the history
    buffer holds ctx + 1 ids, and the stream equals the oracle's."""
    from aotk import configs
    spec = configs.build("tiny-llama")
    blob = oracle.synth_blob(spec, 0x5EED)
    ctx = 12
    gm = aotk.Model(spec, blob)
    st = aotk.State(gm, ctx)
    ref = oracle.Model(spec, blob, ctx)
    st.forward(5, 0, True)
    ref.forward(5, 0, True)
    got = st.generate(0, ctx + 1)
    assert len(got) == ctx + 1
    assert got == ref.generate(0, ctx + 1)
    # one token more does not fit
    with pytest.raises(aotk.AotkError):
        st.generate(0, ctx + 2)
