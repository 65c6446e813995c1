"""The five benchmark configs' greedy token streams at their written lengths,
on the GPU, against the oracle-written fixtures of tests/golden/stream_*.npz
(tests/golden/make_streams.py): the prompt through the batched prompt loop
in 64-token chunks (crates/aot-kernels/src/app.rs:474-485), then the greedy
loop (app.rs:553-610) on the device. Token ids must be identical, and the
prompt-end and last-step logits bit for bit (SHA-256 of the f32 bytes).

    configs[0] TinyLlama-1.1B Q4_K_M:    6-token prompt,   32 greedy tokens
    configs[2] Llama-3-8B Q4_K_M:      512-token prompt,  128 greedy tokens
    configs[3] Qwen3-8B Q8_0:         4096-token prefill, 256 greedy tokens
    configs[4] Gemma-3-4B Q5_K_M:     8192-token prefill, 256 greedy tokens
"""
import hashlib
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
NAMES = ["tinyllama-1.1b-q4km", "llama3-8b-q4km", "qwen3-8b-q8_0", "gemma3-4b-q5km"]


def _fixture(name):
    path = os.path.join(GOLDEN, f"stream_{name}.npz")
    if not os.path.exists(path):
        pytest.fail(f"missing fixture {path}: run tests/golden/make_streams.py")
    return np.load(path)


def _sha(logits):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(logits, np.float32).tobytes()).digest(), np.uint8)


def _top(f, which, logits):
    ids = f[f"{which}_top_ids"]
    return f"fixture top ids {ids[:4].tolist()} vals {f[f'{which}_top_vals'][:4].tolist()}; " \
           f"got vals at those ids {logits[ids[:4]].tolist()}, argmax {int(np.argmax(logits))}"


@pytest.mark.gpu
@pytest.mark.parametrize("name", NAMES)
def test_config_stream_full_length(aotk, name):
    from aotk import configs
    f = _fixture(name)
    prompt = [int(t) for t in f["prompt"]]
    want = [int(t) for t in f["greedy"]]
    chunk = int(f["chunk"])
    print(f"[stream] {name}: {len(prompt)} prompt tokens, {len(want)} greedy", flush=True)
    spec = configs.build(name)
    gm = aotk.Model(spec, seed=0x5EED)
    st = aotk.State(gm, len(prompt) + len(want), chunk)
    try:
        st.prompt(prompt, batch=chunk)
        lp = st.logits()
        assert np.array_equal(_sha(lp), f["prompt_sha256"]), f"{name}: prompt-end logits differ; " + _top(f, "prompt", lp)
        got = st.generate(len(prompt), len(want))
        first = next((i for i, (a, b) in enumerate(zip(got, want)) if a != b), None)
        assert got == want, f"{name}: greedy streams part at token {first}: {got[first:first + 4]} vs {want[first:first + 4]}"
        lf = st.logits()
        assert np.array_equal(_sha(lf), f["final_sha256"]), f"{name}: last-step logits differ; " + _top(f, "final", lf)
    finally:
        st.free()
        gm.free()


@pytest.mark.gpu
def test_prefix_continuation_at_config_scale(aotk):
    """--save-kv / --load-kv (prefix.rs, app.rs:458-489) at the Qwen3-8B
    config's size: 4095 prompt positions saved to an AOTP blob (1.2 GB),
    loaded into a fresh state, the last prompt token evaluated there, then
    256 greedy tokens: the stream and both logits digests equal the
    uninterrupted run's fixture."""
    from aotk import configs
    f = _fixture("qwen3-8b-q8_0")
    prompt = [int(t) for t in f["prompt"]]
    want = [int(t) for t in f["greedy"]]
    spec = configs.build("qwen3-8b-q8_0")
    gm = aotk.Model(spec, seed=0x5EED)
    ctx = len(prompt) + len(want)
    a = aotk.State(gm, ctx, 64)
    try:
        a.prompt(prompt[:-1], batch=64)
        blob = a.save_prefix(prompt, len(prompt) - 1)
    finally:
        a.free()
    b = aotk.State(gm, ctx, 64)
    try:
        toks, nc = b.load_prefix(blob)
        assert toks == prompt and nc == len(prompt) - 1
        b.forward(prompt[-1], nc, True)
        assert np.array_equal(_sha(b.logits()), f["prompt_sha256"])
        assert b.generate(len(prompt), len(want)) == want
        assert np.array_equal(_sha(b.logits()), f["final_sha256"])
    finally:
        b.free()
        gm.free()


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["tinyllama-1.1b-q4km", "llama3-8b-q4km", "qwen3-8b-q8_0", "gemma3-4b-q5km"])
def test_config_sampled_stream(aotk, name):
    """The sampled loop (app.rs:553-610 with sampler.rs: temperature 0.8,
    top-k 40, top-p 0.95, repeat penalty 1.1 over a 64-token window, seed
    42) on the device at the config's written length (Qwen3: after the
    4096-token prefill, Gemma-3 after the 8192-token one, 256 sampled
    tokens), against the
    oracle-written fixture (tests/golden/make_streams.py --sampled)."""
    from aotk import configs
    path = os.path.join(GOLDEN, f"sampled_{name}.npz")
    if not os.path.exists(path):
        pytest.fail(f"missing fixture {path}: run tests/golden/make_streams.py --sampled")
    f = np.load(path)
    prompt = [int(t) for t in f["prompt"]]
    want = [int(t) for t in f["sampled"]]
    cfg = dict(temperature=float(f["temperature"]), top_k=int(f["top_k"]), top_p=float(f["top_p"]),
               repeat_penalty=float(f["repeat_penalty"]), repeat_last_n=int(f["repeat_last_n"]), seed=int(f["seed"]))
    spec = configs.build(name)
    gm = aotk.Model(spec, seed=0x5EED)
    st = aotk.State(gm, len(prompt) + len(want), int(f["chunk"]))
    sp = aotk.Sampler(**cfg)
    try:
        st.prompt(prompt, batch=int(f["chunk"]))
        got = st.generate_sampled(sp, len(prompt), len(want), prompt)
        first = next((i for i, (a, b) in enumerate(zip(got, want)) if a != b), None)
        assert got == want, f"{name}: sampled streams part at token {first}"
    finally:
        sp.free()
        st.free()
        gm.free()
