"""KV prefix blobs "AOTP" v2 (crates/aot-kernels/src/prefix.rs): the oracle's
restatement of the format on the CPU (layout, padding, the checks of
Prefix::parse), then the library's save / load through the C-ABI against it,
and a saved run continued in a fresh state (--save-kv / --load-kv,
app.rs:397-489, 631-632)."""
import numpy as np
import pytest

L, KV = 3, 16


def _kv(ctx, seed=0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(L * ctx * KV).astype(np.float32), rng.standard_normal(L * ctx * KV).astype(np.float32))


def test_layout_and_padding(oracle):
    ctx = 12
    k, v = _kv(ctx)
    for n, data_off in ((10, 64), (11, 128), (1, 64), (26, 128)):
        toks = list(range(100, 100 + n))
        nc = min(n, 7)
        b = oracle.prefix_serialize(k, v, ctx, L, KV, toks, nc)
        assert b[:4] == b"AOTP"
        assert np.frombuffer(b[4:24], "<u4").tolist() == [2, n, L, KV, nc]
        assert np.frombuffer(b[24:24 + 4 * n], "<u4").tolist() == toks
        assert all(x == 0 for x in b[24 + 4 * n:data_off])
        assert len(b) == data_off + L * 2 * nc * KV * 4
        # layer 1's V rows sit after layer 0's K, V and layer 1's K
        rows = nc * KV * 4
        v1 = np.frombuffer(b[data_off + 3 * rows:data_off + 4 * rows], "<f4").reshape(nc, KV)
        assert np.array_equal(v1, v.reshape(L, ctx, KV)[1, :nc])


def test_round_trip_and_clamp(oracle):
    ctx = 9
    k, v = _kv(ctx, 1)
    toks = [5, 6, 7, 8]
    b = oracle.prefix_serialize(k, v, ctx, L, KV, toks, 99)  # n_cached clamps to n (prefix.rs:117)
    t, nc, kr, vr = oracle.prefix_parse(b, L, KV)
    assert t == toks and nc == 4
    assert np.array_equal(kr, k.reshape(L, ctx, KV)[:, :4]) and np.array_equal(vr, v.reshape(L, ctx, KV)[:, :4])


def test_parse_rejects(oracle):
    ctx = 6
    k, v = _kv(ctx, 2)
    good = oracle.prefix_serialize(k, v, ctx, L, KV, [1, 2, 3], 2)
    assert oracle.prefix_parse(good, L, KV) is not None

    def patch(at, val):
        b = bytearray(good)
        b[at:at + 4] = np.array([val], "<u4").tobytes()
        return bytes(b)

    bad = {
        "short": good[:23],
        "magic": b"AOTQ" + good[4:],
        "version": patch(4, 3),
        "layers": patch(12, L + 1),
        "kv_dim": patch(16, KV * 2),
        "empty": patch(8, 0),
        "n_cached > n": patch(20, 4),
        "truncated": good[:-1],
    }
    for name, b in bad.items():
        assert oracle.prefix_parse(b, L, KV) is None, name
    # version 1: n_cached is n_tokens whatever the field holds
    v1 = oracle.prefix_serialize(k, v, ctx, L, KV, [1, 2, 3], 3)
    v1 = bytearray(v1)
    v1[4:8] = np.array([1], "<u4").tobytes()
    v1[20:24] = np.array([0], "<u4").tobytes()
    t, nc, _, _ = oracle.prefix_parse(bytes(v1), L, KV)
    assert t == [1, 2, 3] and nc == 3


def _pair(aotk, oracle, name, ctx):
    from aotk import configs
    spec = configs.build(name)
    blob = oracle.synth_blob(spec, 0x5EED)
    return spec, blob, aotk.Model(spec, blob), oracle.Model(spec, blob, ctx)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["tiny-llama", "tiny-gemma3"])
def test_save_matches_oracle_bytes(aotk, oracle, name):
    from aotk import configs
    ctx = 40
    spec, _, gm, ref = _pair(aotk, oracle, name, ctx)
    d = spec.d
    kv = d["n_kv_head"] * d["head_dim"]
    toks = configs.prompt_tokens(11, 13, d["vocab"])
    st = aotk.State(gm, ctx)
    st.prompt(toks)
    ref.prompt(toks)
    k, v = ref.kv(ctx)
    for n_cached in (13, 12, 1):
        want = oracle.prefix_serialize(k, v, ctx, d["n_layer"], kv, toks, n_cached)
        assert st.save_prefix(toks, n_cached) == want, n_cached


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["tiny-llama", "tiny-q4km"])
def test_load_and_continue(aotk, oracle, name):
    """A saved run whose last token was never fed back (n_cached = n - 1),
    loaded into a fresh state and continued, equals the uninterrupted run."""
    from aotk import configs
    ctx = 48
    spec, _, gm, ref = _pair(aotk, oracle, name, ctx)
    d = spec.d
    kv = d["n_kv_head"] * d["head_dim"]
    toks = configs.prompt_tokens(5, 10, d["vocab"])
    ref.prompt(toks)
    gen = ref.generate(len(toks), 6)        # tokens at positions 10..15; the last is not fed back
    run = toks + gen
    k, v = ref.kv(ctx)
    blob = oracle.prefix_serialize(k, v, ctx, d["n_layer"], kv, run, len(run) - 1)
    more = configs.prompt_tokens(6, 5, d["vocab"])
    full = run + more
    # reference: the uninterrupted sequence evaluated from scratch
    ref2 = oracle.Model(spec, oracle.synth_blob(spec, 0x5EED), ctx)
    ref2.prompt(full, batch=4)
    want_logits = ref2.logits()
    want_gen = ref2.generate(len(full), 5)
    st = aotk.State(gm, ctx)
    got_toks, nc = st.load_prefix(blob)
    assert got_toks == run and nc == len(run) - 1
    k2, v2 = st.kv_download(nc)
    assert np.array_equal(k2.reshape(d["n_layer"], nc, kv), k.reshape(d["n_layer"], ctx, kv)[:, :nc])
    assert np.array_equal(v2.reshape(d["n_layer"], nc, kv), v.reshape(d["n_layer"], ctx, kv)[:, :nc])
    # evaluate the rest like app.rs:474-485 from `cached` on
    rest = full[nc:]
    done = nc
    while done < len(full):
        end = min(done + 4, len(full))
        if end - done == 1:
            st.forward(full[done], done, end == len(full))
        else:
            st.forward_batch(full[done:end], done, end == len(full))
        done = end
    assert np.array_equal(st.logits(), want_logits)
    assert st.generate(len(full), 5) == want_gen
    assert len(rest) == len(more) + 1


@pytest.mark.gpu
def test_load_rejects(aotk, oracle):
    from aotk import configs
    ctx = 16
    spec, _, gm, _ = _pair(aotk, oracle, "tiny-llama", ctx)
    d = spec.d
    kv = d["n_kv_head"] * d["head_dim"]
    k = np.zeros(d["n_layer"] * ctx * kv, np.float32)
    good = oracle.prefix_serialize(k, k, ctx, d["n_layer"], kv, [1, 2, 3], 3)
    st = aotk.State(gm, ctx)
    assert st.load_prefix(good) == ([1, 2, 3], 3)
    too_long = oracle.prefix_serialize(np.zeros(d["n_layer"] * 20 * kv, np.float32), np.zeros(d["n_layer"] * 20 * kv, np.float32),
                                       20, d["n_layer"], kv, list(range(20)), 20)
    other = oracle.prefix_serialize(np.zeros((d["n_layer"] + 1) * ctx * kv, np.float32), np.zeros((d["n_layer"] + 1) * ctx * kv, np.float32),
                                    ctx, d["n_layer"] + 1, kv, [1], 1)
    for b in (good[:20], b"XXXX" + good[4:], good[:-4], other, too_long, b""):
        with pytest.raises(aotk.AotkError):
            st.load_prefix(b)
