"""The benchmark model shapes on the GPU against the oracle, bit for bit:
greedy streams after a short prompt (batched prompt path) for the Llama-3-8B,
Qwen3-8B and Gemma-3-4B configs, and single decode steps at the long
contexts of the Qwen3 (4096 positions) and Gemma-3 (8192 positions, sliding
window 1024 on local layers) configs with a random KV cache loaded into both.
The TinyLlama config is covered in test_gpu_model.py."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _pair(aotk, oracle, name, ctx, max_batch):
    from aotk import configs
    spec = configs.build(name)
    gm = aotk.Model(spec, seed=0x5EED)
    blob = gm.download()  # the same bytes for both sides
    st = aotk.State(gm, ctx, max_batch)
    ref = oracle.Model(spec, blob, ctx, max_batch=max_batch, n_threads=16)
    return spec, gm, st, ref


@pytest.mark.parametrize("name", ["llama3-8b-q4km", "qwen3-8b-q8_0", "gemma3-4b-q5km"])
def test_config_prompt_and_greedy(aotk, oracle, name):
    from aotk import configs
    n_prompt, n_gen = 20, 6
    spec, gm, st, ref = _pair(aotk, oracle, name, n_prompt + n_gen + 1, 32)
    toks = configs.prompt_tokens(1, n_prompt, spec.d["vocab"])
    st.prompt(toks, batch=32)
    ref.prompt(toks, batch=32)
    a, b = st.logits(), ref.logits()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{name}: prompt logits differ"
    assert st.generate(n_prompt, n_gen) == ref.generate(n_prompt, n_gen)
    # the last decode step's logits, bit for bit
    assert np.array_equal(st.logits().view(np.uint32), ref.logits().view(np.uint32)), f"{name}: decode logits differ"
    ref.close()
    st.free()
    gm.free()


@pytest.mark.parametrize("name", ["llama3-8b-q4km", "gemma3-4b-q5km"])
def test_config_full_prompt_chunk(aotk, oracle, name):
    """A full 64-token prompt chunk and a ragged one (70 tokens in batches
    of 64) at the real shapes: four token tiles through the prompt matmuls,
    including the launch that runs q/k and v (different kinds) together."""
    from aotk import configs
    n_prompt = 70
    spec, gm, st, ref = _pair(aotk, oracle, name, n_prompt + 1, 64)
    toks = configs.prompt_tokens(2, n_prompt, spec.d["vocab"])
    st.prompt(toks, batch=64)
    ref.prompt(toks, batch=64)
    a, b = st.logits(), ref.logits()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{name}: prompt logits differ"
    ref.close()
    st.free()
    gm.free()


@pytest.mark.parametrize("name,n_pos", [("qwen3-8b-q8_0", 4096), ("gemma3-4b-q5km", 8192)])
def test_config_long_context_decode(aotk, oracle, name, n_pos):
    spec, gm, st, ref = _pair(aotk, oracle, name, n_pos + 2, 1)
    d = spec.d
    kv = d["n_kv_head"] * d["head_dim"]
    rng = np.random.default_rng(n_pos)
    k = (rng.standard_normal((d["n_layer"], n_pos, kv)) * 0.5).astype(np.float32)
    v = rng.standard_normal((d["n_layer"], n_pos, kv)).astype(np.float32)
    st.kv_upload(n_pos, k, v)
    rk, rv = ref.kv(n_pos + 2)
    rk.reshape(d["n_layer"], n_pos + 2, kv)[:, :n_pos] = k
    rv.reshape(d["n_layer"], n_pos + 2, kv)[:, :n_pos] = v
    tok = 7
    st.forward(tok, n_pos, True)
    ref.forward(tok, n_pos, True)
    a, b = st.logits(), ref.logits()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"{name}: decode logits at {n_pos} differ"
    t1 = int(np.argmax(a))
    st.forward(t1, n_pos + 1, True)
    ref.forward(t1, n_pos + 1, True)
    assert np.array_equal(st.logits().view(np.uint32), ref.logits().view(np.uint32))
    ref.close()
    st.free()
    gm.free()
