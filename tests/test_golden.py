"""Golden fixtures (tests/golden/, written by make_golden.py from the pinned
oracle): the oracle still reproduces them (CPU), and the HIP path reproduces
them bit for bit (GPU)."""
import os

import numpy as np
import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KINDS = {"F32": 0, "F16": 1, "BF16": 2, "Q4_0": 3, "Q5_0": 4, "Q8_0": 5, "Q4_K": 6, "Q5_K": 7, "Q6_K": 8}
MODELS = ("tiny-llama", "tiny-q4km", "tiny-q8_0", "tiny-q5km")


def load(name):
    return np.load(os.path.join(HERE, name), allow_pickle=False)


def act_of(oracle, kind, f, name):
    xq = f[f"{name}_xq"]
    if kind in (3, 4, 5):
        return np.frombuffer(xq.tobytes(), oracle.Q8_0_DTYPE)
    if kind in (6, 7, 8):
        return np.frombuffer(xq.tobytes(), oracle.Q8_K_DTYPE)
    return f[f"{name}_x"]


@pytest.mark.parametrize("name", list(KINDS))
def test_oracle_reproduces_matvec_fixture(oracle, name):
    kind = KINDS[name]
    f = load("matvec_512.npz")
    x = f[f"{name}_x"]
    assert np.array_equal(oracle.quantize_rows(kind, np.zeros((1, 512), np.float32)).shape[1],
                          f[f"{name}_w"].shape[1])
    xa = oracle.quantize_act(kind, x)
    assert xa.tobytes() == act_of(oracle, kind, f, name).tobytes()
    assert np.array_equal(oracle.dequant_rows(kind, f[f"{name}_w"], 512), f[f"{name}_deq"])
    y = oracle.matvec(kind, f[f"{name}_w"], xa, 3, 512)
    assert np.array_equal(y.view(np.uint32), f[f"{name}_y"].view(np.uint32))


@pytest.mark.parametrize("name", MODELS)
def test_oracle_reproduces_model_fixture(oracle, name):
    from aotk import configs
    f = load(f"model_{name}.npz")
    spec = configs.build(name)
    blob = oracle.synth_blob(spec, 0x5EED)
    m = oracle.Model(spec, blob, 32, max_batch=8, n_threads=4)
    m.prompt([int(t) for t in f["prompt"]], batch=8)
    assert np.array_equal(m.logits().view(np.uint32), f["logits"].view(np.uint32))
    assert m.generate(6, 16) == [int(t) for t in f["greedy"]]
    m.close()


@pytest.mark.gpu
@pytest.mark.parametrize("name", list(KINDS))
def test_gpu_matches_matvec_fixture(aotk, oracle, name):
    kind = KINDS[name]
    f = load("matvec_512.npz")
    w = aotk.Weight(kind, f[f"{name}_w"], 3, 512)
    assert np.array_equal(aotk.dequant_rows(w), f[f"{name}_deq"])
    y = aotk.matvec(w, act_of(oracle, kind, f, name))
    assert np.array_equal(y.view(np.uint32), f[f"{name}_y"].view(np.uint32))
    y2 = aotk.matvec_f32(w, f[f"{name}_x"])
    assert np.array_equal(y2.view(np.uint32), f[f"{name}_y"].view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("name", MODELS)
def test_gpu_matches_model_fixture(aotk, name):
    from aotk import configs
    f = load(f"model_{name}.npz")
    spec = configs.build(name)
    m = aotk.Model(spec, seed=0x5EED)
    st = aotk.State(m, 32, 8)
    st.prompt([int(t) for t in f["prompt"]], batch=8)
    assert np.array_equal(st.logits().view(np.uint32), f["logits"].view(np.uint32))
    assert st.generate(6, 16) == [int(t) for t in f["greedy"]]


STREAMS = {"tinyllama-1.1b-q4km": (1, 6, 32), "llama3-8b-q4km": (1, 512, 128),
           "qwen3-8b-q8_0": (2, 4096, 256), "gemma3-4b-q5km": (2, 8192, 256)}


@pytest.mark.parametrize("name", list(STREAMS))
def test_stream_fixture_shape(name):
    """The full-length stream fixtures hold the config's own prompt (the
    seeded splitmix64 ids bench.py uses) and stream length."""
    from aotk import configs
    seed, n_prompt, n_gen = STREAMS[name]
    f = load(f"stream_{name}.npz")
    vocab = configs.build(name).d["vocab"]
    assert f["prompt"].tolist() == configs.prompt_tokens(seed, n_prompt, vocab)
    assert f["greedy"].shape == (n_gen,) and int(f["greedy"].max()) < vocab
    assert int(f["chunk"]) == 64 and f["prompt_sha256"].shape == (32,)


def test_oracle_reproduces_tinyllama_stream(oracle):
    """configs[0] is small enough to recompute here: the oracle still
    writes the committed stream and logits digests."""
    import hashlib
    from aotk import configs
    f = load("stream_tinyllama-1.1b-q4km.npz")
    spec = configs.build("tinyllama-1.1b-q4km")
    blob = oracle.synth_blob(spec, 0x5EED)
    m = oracle.Model(spec, blob, 38, max_batch=64, n_threads=8)
    m.prompt([int(t) for t in f["prompt"]], batch=64)
    sha = lambda a: np.frombuffer(hashlib.sha256(a.tobytes()).digest(), np.uint8)  # noqa: E731
    assert np.array_equal(sha(m.logits()), f["prompt_sha256"])
    assert m.generate(6, 32) == f["greedy"].tolist()
    assert np.array_equal(sha(m.logits()), f["final_sha256"])
    m.close()


@pytest.mark.parametrize("name,seed,n_prompt,n_gen", [("tinyllama-1.1b-q4km", 1, 6, 32), ("llama3-8b-q4km", 1, 512, 128),
                                                   ("qwen3-8b-q8_0", 2, 4096, 256),
                                                   ("gemma3-4b-q5km", 2, 8192, 256)])
def test_sampled_fixture_shape(name, seed, n_prompt, n_gen):
    from aotk import configs
    f = load(f"sampled_{name}.npz")
    vocab = configs.build(name).d["vocab"]
    assert f["prompt"].tolist() == configs.prompt_tokens(seed, n_prompt, vocab)
    assert f["sampled"].shape == (n_gen,) and int(f["sampled"].max()) < vocab
    assert float(f["temperature"]) == 0.8 and int(f["top_k"]) == 40 and int(f["seed"]) == 42


def test_oracle_reproduces_tinyllama_sampled_stream(oracle):
    from aotk import configs
    f = load("sampled_tinyllama-1.1b-q4km.npz")
    spec = configs.build("tinyllama-1.1b-q4km")
    blob = oracle.synth_blob(spec, 0x5EED)
    m = oracle.Model(spec, blob, 38, max_batch=64, n_threads=8)
    toks = [int(t) for t in f["prompt"]]
    m.prompt(toks, batch=64)
    cfg = dict(temperature=0.8, top_k=40, top_p=0.95, repeat_penalty=1.1, repeat_last_n=64, seed=42)
    assert m.generate_sampled(6, 32, oracle.Sampler(**cfg), toks) == f["sampled"].tolist()
    m.close()
