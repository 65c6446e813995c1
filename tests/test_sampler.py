"""Stochastic sampler (crates/aot-kernels/src/sampler.rs).

CPU: the oracle's restatement against the reference's own unit tests
(sampler.rs:120-147), the published first SplitMix64 output, and the
distribution the draw must follow. GPU: the device sampler through the C-ABI
against the oracle, token for token over successive draws (the xorshift64*
stream advances on both sides), and the sampled generation loop of a model.

Candidates of equal scaled logit are taken in ascending token id on both
sides; the reference's unstable sort leaves that order open, so a tie that
straddles the sampled point is parity unpinned."""
import numpy as np
import pytest


def test_reference_unit_tests(oracle):
    # greedy_picks_max (sampler.rs:124-129)
    assert oracle.Sampler().sample(np.array([0.1, 5.0, 2.0], np.float32)) == 1
    # temperature_sampling_respects_top_k (:131-140)
    s = oracle.Sampler(temperature=1.0, top_k=2, top_p=1.0, seed=7)
    for _ in range(200):
        assert s.sample(np.array([0.0, 10.0, 9.0, -5.0], np.float32)) in (1, 2)
    # repeat_penalty_lowers_recent (:142-147)
    s = oracle.Sampler(repeat_penalty=100.0)
    assert s.sample(np.array([1.0, 1.1], np.float32), [1]) == 0


def test_splitmix_seed(oracle):
    # SplitMix64's first output for state 0 is 0xE220A8397B1DCDAF (odd already)
    assert oracle.load().or_sampler_seed(0) == 0xE220A8397B1DCDAF


def test_distribution_and_top_p(oracle):
    p = np.array([0.5, 0.3, 0.2], np.float64)
    logits = np.log(p).astype(np.float32)
    # top_p 0.75 keeps {0, 1} (0.5 < 0.75 <= 0.8) renormalised to 0.625 / 0.375
    s = oracle.Sampler(temperature=1.0, top_k=0, top_p=0.75, seed=3)
    draws = [s.sample(logits.copy()) for _ in range(4000)]
    assert set(draws) == {0, 1}
    assert abs(draws.count(0) / 4000 - 0.625) < 0.03
    # no cut: the softmax probabilities
    s = oracle.Sampler(temperature=1.0, top_k=0, top_p=1.0, seed=4)
    draws = np.array([s.sample(logits.copy()) for _ in range(6000)])
    freq = np.bincount(draws, minlength=3) / 6000
    assert np.abs(freq - p).max() < 0.03
    # temperature 0.5 squares the odds
    s = oracle.Sampler(temperature=0.5, top_k=0, top_p=1.0, seed=5)
    draws = np.array([s.sample(logits.copy()) for _ in range(6000)])
    q = p ** 2 / (p ** 2).sum()
    assert np.abs(np.bincount(draws, minlength=3) / 6000 - q).max() < 0.03


def test_penalty_in_place(oracle):
    lg = np.array([2.0, -2.0, 1.0, 0.5], np.float32)
    s = oracle.Sampler(temperature=0.0, repeat_penalty=2.0, repeat_last_n=3)
    # window = last 3 of [2, 0, 1, 1]: token 1 twice, token 0 once
    assert s.sample(lg, [2, 0, 1, 1]) == 0  # first of the tied maxima
    assert lg.tolist() == [1.0, -8.0, 1.0, 0.5]


CASES = [
    dict(temperature=0.8, top_k=40, top_p=0.95, seed=7),
    dict(temperature=1.0, top_k=1, top_p=1.0, seed=1),
    dict(temperature=1.3, top_k=1024, top_p=0.5, seed=11),
    dict(temperature=0.7, top_k=300, top_p=1.0, repeat_penalty=1.3, repeat_last_n=64, seed=99),
    dict(temperature=0.0, top_k=40, top_p=0.95, repeat_penalty=1.5, repeat_last_n=8, seed=5),
    dict(temperature=2.0, top_k=0, top_p=0.9, seed=4242),  # top_k 0: the whole (small) vocab
]


@pytest.mark.gpu
@pytest.mark.parametrize("vocab", [512, 32000, 151936, 262144])
def test_device_sampler_matches_oracle(aotk, oracle, vocab):
    from aotk import configs
    spec = configs.build(dict(configs.TEST_CONFIGS["tiny-llama"], vocab=vocab))
    gm = aotk.Model(spec, seed=2)
    st = aotk.State(gm, 8, 1)
    rng = np.random.default_rng(vocab)
    for ci, cfg in enumerate(CASES):
        if cfg.get("top_k") == 0 and cfg["temperature"] > 0 and vocab > 1024:
            continue
        ds = aotk.Sampler(**cfg)
        os_ = oracle.Sampler(**cfg)
        recent = rng.integers(0, vocab, 40).tolist()
        recent += recent[:5]  # duplicates compound
        for draw in range(12):
            lg = (rng.standard_normal(vocab) * 3).astype(np.float32)
            if draw % 4 == 1:
                lg[rng.integers(0, vocab, 50)] = lg.max()  # ties at the top
            if draw % 4 == 2:
                lg[:vocab // 2] = -np.inf
            want = os_.sample(lg.copy(), recent)
            st.set_logits(lg)
            got = st.sample(ds, recent)
            assert got == want, (vocab, ci, draw, got, want)
        ds.free()


@pytest.mark.gpu
def test_device_sampler_limits(aotk):
    from aotk import configs
    spec = configs.build(dict(configs.TEST_CONFIGS["tiny-llama"], vocab=4096))
    st = aotk.State(aotk.Model(spec, seed=2), 8, 1)
    st.set_logits(np.zeros(4096, np.float32))
    for cfg in (dict(temperature=1.0, top_k=0), dict(temperature=1.0, top_k=2000)):
        with pytest.raises(aotk.AotkError):
            st.sample(aotk.Sampler(**cfg))
    with pytest.raises(aotk.AotkError):
        aotk.Sampler(repeat_last_n=5000)
    assert st.sample(aotk.Sampler(temperature=0.0, top_k=0)) == 0  # greedy has no limit


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["tiny-llama", "tiny-gemma3"])
def test_sampled_generation(aotk, oracle, name):
    from aotk import configs
    spec = configs.build(name)
    blob = oracle.synth_blob(spec, 0x5EED)
    ctx = 64
    toks = configs.prompt_tokens(9, 7, spec.d["vocab"])
    for cfg in (dict(temperature=0.9, top_k=40, top_p=0.95, repeat_penalty=1.1, seed=3),
                dict(temperature=1.5, top_k=200, top_p=0.8, seed=8)):
        ref = oracle.Model(spec, blob, ctx)
        ref.prompt(toks)
        want = ref.generate_sampled(len(toks), 20, oracle.Sampler(**cfg), toks)
        st = aotk.State(aotk.Model(spec, blob), ctx)
        st.prompt(toks)
        sp = aotk.Sampler(**cfg)
        assert st.generate_sampled(sp, len(toks), 20, toks) == want
        # the same sampler again continues its rng stream on both sides
        ref2 = oracle.Model(spec, blob, ctx)
        os2 = oracle.Sampler(**cfg)
        ref2.prompt(toks)
        ref2.generate_sampled(len(toks), 20, os2, toks)
        ref2.prompt(toks)
        want2 = ref2.generate_sampled(len(toks), 10, os2, toks)
        st.prompt(toks)
        assert st.generate_sampled(sp, len(toks), 10, toks) == want2
