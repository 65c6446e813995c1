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
