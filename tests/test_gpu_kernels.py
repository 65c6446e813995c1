"""Per-kernel parity of the HIP path against the CPU oracle (bit-exact for
integer / dequantization / quantized-dot work, tolerance for float ops)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F32, F16, BF16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K = range(9)
ALL = [F32, F16, BF16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K]
NAMES = dict(zip(ALL, ["f32", "f16", "bf16", "q4_0", "q5_0", "q8_0", "q4_K", "q5_K", "q6_K"]))


def cols_for(kind):
    return {F32: [8, 64, 2053, 4096], F16: [8, 64, 2053, 4096, 11008, 16384], BF16: [12, 64, 2053, 4096, 14336],
            Q4_0: [32, 96, 2048, 4096, 5632, 14336, 16384, 18432], Q5_0: [32, 96, 2048, 4096, 14336, 16384, 18432],
            Q8_0: [32, 96, 2048, 4096, 12288, 14336, 16384, 18432],
            Q4_K: [256, 512, 2048, 3072, 5632, 14336, 17408], Q5_K: [256, 512, 2560, 4096, 10240, 14336],
            Q6_K: [256, 512, 2048, 5632, 10240, 12288, 14336, 17408]}[kind]


def weights(kind, rows, cols, seed, oracle):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    return oracle.quantize_rows(kind, w)


@pytest.mark.parametrize("kind", ALL, ids=lambda k: NAMES[k])
def test_encoder_and_dequant_bitexact(aotk, oracle, kind):
    rng = np.random.default_rng(kind + 1)
    for cols in cols_for(kind)[:3]:
        x = (rng.standard_normal((37, cols)) * 0.5).astype(np.float32)
        ref = oracle.quantize_rows(kind, x)
        got = aotk.quantize_rows(kind, x)
        assert np.array_equal(ref, got), f"{NAMES[kind]} cols={cols}: device encoder differs"
        w = aotk.Weight(kind, ref, 37, cols)
        deq = aotk.dequant_rows(w)
        ref_deq = oracle.dequant_rows(kind, ref, cols)
        assert np.array_equal(deq.view(np.uint32), ref_deq.view(np.uint32)), f"{NAMES[kind]} dequant differs"


def test_f16_all_halves(aotk, oracle):
    h = np.arange(65536, dtype=np.uint16)
    w = aotk.Weight(F16, h.view(np.uint8), 1, 65536)
    got = aotk.dequant_rows(w)[0]
    ref = oracle.dequant_rows(F16, h.view(np.uint8), 65536)[0]
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_activation_quantizers(aotk, oracle):
    rng = np.random.default_rng(5)
    for n in (256, 2048, 5632):
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        x[7] = -x[3] if n > 256 else x[7]  # magnitude tie: first index wins
        x[512 % n:512 % n + 256] = 0.0  # an all-zero block
        a = aotk.quantize_q8_k(x)
        b = oracle.quantize_q8_k(x)
        assert a.tobytes() == b.tobytes()
        if n > 2048:  # an all-NaN block: the magnitude scan never moves off 0 (a zero block)
            xn = x.copy()
            xn[1024:1280] = np.nan
            assert aotk.quantize_q8_k(xn).tobytes() == oracle.quantize_q8_k(xn).tobytes()
        a0 = aotk.quantize_q8_0(x)
        b0 = oracle.quantize_q8_0(x)
        assert a0.tobytes() == b0.tobytes()
        xn = x.copy()
        xn[64:96] = np.nan  # an all-NaN block: fold(0, max) gives d = 0
        xn[100] = np.nan    # and a NaN among finite values never wins the max
        assert aotk.quantize_q8_0(xn).tobytes() == oracle.quantize_q8_0(xn).tobytes()


@pytest.mark.parametrize("kind", ALL, ids=lambda k: NAMES[k])
def test_matvec_bitexact(aotk, oracle, kind):
    rng = np.random.default_rng(100 + kind)
    for cols in cols_for(kind):
        rows = 67
        raw = weights(kind, rows, cols, kind * 7 + cols, oracle)
        x = (rng.standard_normal(cols) * 2).astype(np.float32)
        act = oracle.quantize_act(kind, x)
        ref = oracle.matvec(kind, raw, act, rows, cols)
        w = aotk.Weight(kind, raw, rows, cols)
        got = aotk.matvec(w, act)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), \
            f"{NAMES[kind]} cols={cols}: max diff {np.abs(got - ref).max()}"
        got2 = aotk.matvec_f32(w, x)
        assert np.array_equal(got2.view(np.uint32), ref.view(np.uint32))


MICRO_KINDS = [Q4_K, Q5_K, Q6_K, Q8_0, Q4_0, Q5_0, F16, BF16]
MICRO_SHAPES = [(4096, 4096), (14336, 4096), (4096, 14336), (128256, 4096)]


@pytest.mark.parametrize("kind", MICRO_KINDS, ids=lambda k: NAMES[k])
def test_matvec_microbench_shapes(aotk, oracle, kind):
    """Every cell of the configs[1] microbench (8 kinds x 4 shapes, the
    lm-head included) bit-exact against the oracle. The rows are 509 distinct
    encoded rows repeated (the kernels' row mapping and launch shape are those
    of the full matrix; only the host encoding is shortened)."""
    rng = np.random.default_rng(200 + kind)
    pool = oracle.Pool(16)
    for rows, cols in MICRO_SHAPES:
        base = weights(kind, 509, cols, kind * 11 + cols, oracle)
        raw = np.resize(base, (rows, base.shape[1]))
        x = (rng.standard_normal(cols)).astype(np.float32)
        act = oracle.quantize_act(kind, x)
        ref = oracle.matvec(kind, raw, act, rows, cols, pool=pool)
        w = aotk.Weight(kind, raw, rows, cols)
        got = aotk.matvec(w, act)
        w.free()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), \
            f"{NAMES[kind]} {rows}x{cols}: {int((got != ref).sum())} rows differ"


@pytest.mark.parametrize("kind", [F16, BF16], ids=lambda k: NAMES[k])
def test_matvec_half_many_rows(aotk, oracle, kind):
    """The shallow-prefetch variant for matrices of 16384 rows or more, and a
    ragged last block of rows."""
    rng = np.random.default_rng(31)
    rows, cols = 16421, 192
    raw = weights(kind, rows, cols, 5, oracle)
    x = (rng.standard_normal(cols) * 2).astype(np.float32)
    act = oracle.quantize_act(kind, x)
    ref = oracle.matvec(kind, raw, act, rows, cols)
    got = aotk.matvec(aotk.Weight(kind, raw, rows, cols), act)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("kind", [Q4_K, Q6_K, Q8_0, Q5_K, F16], ids=lambda k: NAMES[k])
def test_matmul_equals_matvec(aotk, oracle, kind):
    rng = np.random.default_rng(7)
    cols, rows = 512, 37
    raw = weights(kind, rows, cols, 3, oracle)
    w = aotk.Weight(kind, raw, rows, cols)
    for m in (1, 3, 4, 7, 9):
        xs = [(rng.standard_normal(cols)).astype(np.float32) for _ in range(m)]
        acts = np.concatenate([oracle.quantize_act(kind, x) for x in xs])
        got = aotk.matmul(w, acts, m)
        ref = oracle.matmul(kind, raw, acts, m, rows, cols).reshape(m, rows)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("kind", ALL, ids=lambda k: NAMES[k])
def test_matmul_batched_every_kind(aotk, oracle, kind):
    """The batched prompt kernels of every kind (matvec.rs:524-546, the x4
    kernels simd_avx2.rs:273-430) equal m matvecs bit for bit: ragged row
    counts, batches past one 64-token grid row, odd float widths (scalar
    tail), widths above 16384 columns."""
    rng = np.random.default_rng(70 + kind)
    widths = {F32: [8, 2053, 4096], F16: [64, 2053, 4104], BF16: [12, 2050, 4096], Q4_0: [32, 2048, 18432],
              Q5_0: [96, 4096, 14336], Q8_0: [32, 4096, 18432], Q4_K: [256, 4096], Q5_K: [512, 2560], Q6_K: [256, 5632]}[kind]
    for cols in widths:
        rows = 75
        raw = weights(kind, rows, cols, cols + kind, oracle)
        w = aotk.Weight(kind, raw, rows, cols)
        for m in (2, 17, 64, 100):
            xs = [(rng.standard_normal(cols)).astype(np.float32) for _ in range(m)]
            acts = np.concatenate([oracle.quantize_act(kind, x) for x in xs])
            got = aotk.matmul(w, acts, m)
            ref = oracle.matmul(kind, raw, acts, m, rows, cols, pool=oracle.Pool(8)).reshape(m, rows)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (cols, m)
            if m == 17:  # and the matvec of one of the tokens
                one = aotk.matvec(w, oracle.quantize_act(kind, xs[5]))
                assert np.array_equal(one.view(np.uint32), ref[5].view(np.uint32)), cols
        w.free()


@pytest.mark.parametrize("kind,rows,cols", [(Q8_0, 6144, 4096), (Q8_0, 4096, 12288)], ids=["qkv", "down"])
def test_matmul_qwen3_layer_chunk(aotk, oracle, kind, rows, cols):
    """A 64-token prompt chunk through the Qwen3-8B Q8_0 layer shapes
    (configs[3]; q/k/v fused to 6144 rows), bit-exact (509 rows tiled)."""
    rng = np.random.default_rng(rows + cols)
    m = 64
    base = weights(kind, 509, cols, rows, oracle)
    raw = np.resize(base, (rows, base.shape[1]))
    w = aotk.Weight(kind, raw, rows, cols)
    xs = [(rng.standard_normal(cols)).astype(np.float32) for _ in range(m)]
    acts = np.concatenate([oracle.quantize_act(kind, x) for x in xs])
    got = aotk.matmul(w, acts, m)
    ref = oracle.matmul(kind, raw, acts, m, rows, cols, pool=oracle.Pool(16)).reshape(m, rows)
    w.free()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("kind", [Q4_K, Q5_K, Q6_K], ids=lambda k: NAMES[k])
def test_matmul_many_rows(aotk, oracle, kind):
    """2048 rows or more take the whole batch per 16-row block (super-blocks
    split over the waves): ragged row and token counts, a tile boundary."""
    rng = np.random.default_rng(17)
    cols, rows = 1280, 2100
    raw = weights(kind, rows, cols, 9, oracle)
    w = aotk.Weight(kind, raw, rows, cols)
    for m in (2, 17, 64):
        xs = [(rng.standard_normal(cols)).astype(np.float32) for _ in range(m)]
        acts = np.concatenate([oracle.quantize_act(kind, x) for x in xs])
        got = aotk.matmul(w, acts, m)
        ref = oracle.matmul(kind, raw, acts, m, rows, cols).reshape(m, rows)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), m


def random_kquant_rows(kind, rows, cols, rng):
    """K-quant rows of uniformly random bytes (every quant and every 6-bit
    scale and min value, 63 included) with d = dmin = 2^-6: the edge of the
    prompt kernels' exact integer ranges (quant x scale part products,
    int32 sums)."""
    sb = cols // 256
    size = {Q4_K: 144, Q5_K: 176, Q6_K: 210}[kind]
    raw = rng.integers(0, 256, size=(rows, sb, size), dtype=np.uint8)
    half = np.frombuffer(np.float16(2.0 ** -6).tobytes(), dtype=np.uint8)
    if kind == Q6_K:
        raw[:, :, 208:210] = half  # d after ql, qh and the 16 scales
    else:
        raw[:, :, 0:2] = half      # d
        raw[:, :, 2:4] = half      # dmin
    return raw.reshape(rows, sb * size)


@pytest.mark.parametrize("kind", [Q4_K, Q5_K, Q6_K], ids=lambda k: NAMES[k])
def test_matmul_kquant_extreme_values(aotk, oracle, kind):
    """Random-byte K-quant weights against activations that quantize to
    +-127 in most places, through the whole-batch prompt kernel (2048+
    rows: the scale-folded matrix-core path for Q4_K) and the split one
    (fewer rows), bit-exact, at full and ragged batches."""
    rng = np.random.default_rng(99 + kind)
    cols = 1024
    for rows in (2064, 300):
        raw = random_kquant_rows(kind, rows, cols, rng)
        w = aotk.Weight(kind, raw, rows, cols)
        for m in (64, 40):
            xs = [(np.sign(rng.standard_normal(cols)) * (1.0 + 0.01 * rng.random(cols))).astype(np.float32)
                  for _ in range(m)]
            acts = np.concatenate([oracle.quantize_act(kind, x) for x in xs])
            got = aotk.matmul(w, acts, m)
            ref = oracle.matmul(kind, raw, acts, m, rows, cols, pool=oracle.Pool(8)).reshape(m, rows)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (rows, m)
            one = aotk.matvec(w, oracle.quantize_act(kind, xs[3]))
            assert np.array_equal(one.view(np.uint32), ref[3].view(np.uint32)), (rows, "matvec")
        w.free()


@pytest.mark.parametrize("kind,rows,cols", [(Q4_K, 4096, 4096), (Q4_K, 1024, 4096), (Q6_K, 1024, 4096),
                                            (Q4_K, 14336, 4096), (Q6_K, 4096, 14336)],
                         ids=["wq", "wk", "wv", "gate", "down"])
def test_matmul_llama3_layer_chunk(aotk, oracle, kind, rows, cols):
    """One 64-token prompt chunk through every matrix shape of a Llama-3-8B
    Q4_K_M layer, bit-exact: the 16-row whole-batch kernel at
    4096+ rows and the split kernel at 1024 rows (509 distinct rows tiled)."""
    rng = np.random.default_rng(rows + cols + kind)
    m = 64
    base = weights(kind, 509, cols, rows, oracle)
    raw = np.resize(base, (rows, base.shape[1]))
    w = aotk.Weight(kind, raw, rows, cols)
    xs = [(rng.standard_normal(cols)).astype(np.float32) for _ in range(m)]
    acts = np.concatenate([oracle.quantize_act(kind, x) for x in xs])
    got = aotk.matmul(w, acts, m)
    ref = oracle.matmul(kind, raw, acts, m, rows, cols, pool=oracle.Pool(16)).reshape(m, rows)
    w.free()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_rope_bitexact(aotk, oracle):
    rng = np.random.default_rng(9)
    for neox in (0, 1):
        x = rng.standard_normal(4 * 128).astype(np.float32)
        cs = rng.standard_normal(128).astype(np.float32)
        got = aotk.rope(x, 1, 4, 128, 128, cs, neox)
        ref = x.copy()
        oracle.load().or_rope(oracle.ptr(ref), 4, 128, 128, oracle.ptr(cs), neox)
        assert np.array_equal(got, ref)


def test_rmsnorm_softmax_glu(aotk, oracle):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((3, 2048)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(2048)).astype(np.float32)
    got = aotk.rmsnorm(x, w, 1e-5)
    ref = np.stack([_or_rmsnorm(oracle, r, w) for r in x])
    assert np.array_equal(got, ref)
    s = rng.standard_normal(1000).astype(np.float32) * 4
    ref = s.copy()
    oracle.load().or_softmax(oracle.ptr(ref), ref.size)
    assert np.array_equal(aotk.softmax(s), ref)
    h, up = rng.standard_normal(4096).astype(np.float32), rng.standard_normal(4096).astype(np.float32)
    for fn, name in ((aotk.silu_mul, "or_silu_mul"), (aotk.gelu_mul, "or_gelu_mul")):
        ref = h.copy()
        getattr(oracle.load(), name)(oracle.ptr(ref), oracle.ptr(up), ref.size)
        assert np.array_equal(fn(h, up), ref)


def _or_rmsnorm(oracle, x, w):
    out = np.empty_like(x)
    oracle.load().or_rmsnorm(oracle.ptr(out), oracle.ptr(np.ascontiguousarray(x)), oracle.ptr(w), x.size, 1e-5)
    return out


@pytest.mark.parametrize("hd,nh,nkv,window", [
    (64, 32, 4, 0), (128, 32, 8, 0), (256, 8, 4, 5), (128, 4, 4, 0), (64, 8, 2, 7), (128, 8, 8, 90),
    # every query-heads-per-kv-head ratio at head_dim 256 (1, 2, 4, 8 take the
    # batched-rows scores kernel, 3 and 6 the generic one) and ratio 3 at 64 / 128
    (256, 4, 4, 0), (256, 8, 2, 0), (256, 8, 1, 3), (256, 6, 2, 0), (256, 12, 2, 9),
    (128, 6, 2, 0), (64, 12, 4, 0)])
def test_attention(aotk, oracle, hd, nh, nkv, window):
    rng = np.random.default_rng(hd + nh)
    ctx, layer = 150, 1
    kv = nkv * hd
    kc = rng.standard_normal(2 * ctx * kv).astype(np.float32)
    vc = rng.standard_normal(2 * ctx * kv).astype(np.float32)
    for pos0, m in ((0, 1), (1, 1), (63, 1), (64, 1), (149, 1), (10, 7), (100, 50)):
        q = rng.standard_normal(m * nh * hd).astype(np.float32)
        got = aotk.attention(q, kc, vc, nh, nkv, hd, ctx, layer, pos0, m, window)
        ref = np.zeros(m * nh * hd, np.float32)
        p = oracle.Pool(4)
        oracle.load().or_attention(p.p, oracle.ptr(ref), oracle.ptr(q), oracle.ptr(kc), oracle.ptr(vc), nh, nkv, hd, ctx,
                                   layer, pos0, m, window)
        assert np.array_equal(got, ref), (pos0, m, np.abs(got - ref).max())


@pytest.mark.parametrize("hd,nh,nkv,window,ctx,cases", [
    (128, 32, 8, 0, 4400, ((4300, 1), (2100, 2), (1500, 1), (1980, 64), (4000, 64))),
    (256, 8, 4, 1024, 8300, ((8200, 1), (700, 3), (1000, 40))),
    (256, 8, 4, 0, 8300, ((8200, 1), (5000, 2), (8100, 64))),
])
def test_attention_long_spans(aotk, oracle, hd, nh, nkv, window, ctx, cases):
    """Spans past the one-thread softmax sum (exact parallel replay) and past
    SEQ_MAX_N (sequential fallback); prompt batches up to the per-lane row
    path's 2048-position limit, windowed rows straddling the window edge."""
    rng = np.random.default_rng(hd + ctx)
    kv = nkv * hd
    kc = (rng.standard_normal(ctx * kv) * 0.5).astype(np.float32)
    vc = rng.standard_normal(ctx * kv).astype(np.float32)
    p = oracle.Pool(8)
    for pos0, m in cases:
        q = rng.standard_normal(m * nh * hd).astype(np.float32)
        got = aotk.attention(q, kc, vc, nh, nkv, hd, ctx, 0, pos0, m, window)
        ref = np.zeros(m * nh * hd, np.float32)
        oracle.load().or_attention(p.p, oracle.ptr(ref), oracle.ptr(q), oracle.ptr(kc), oracle.ptr(vc), nh, nkv, hd, ctx,
                                   0, pos0, m, window)
        assert np.array_equal(got, ref), (pos0, m, np.abs(got - ref).max())


def test_argmax(aotk, oracle):
    rng = np.random.default_rng(1)
    x = rng.standard_normal(128256).astype(np.float32)
    assert aotk.argmax(x) == oracle.argmax(x)
    x[5000] = x[90000] = 100.0  # tie: first index wins
    assert aotk.argmax(x) == 5000
    x[3] = np.nan
    assert aotk.argmax(x) == 5000
    assert aotk.argmax(np.full(1000, -np.inf, np.float32)) == 0


def test_libm_matched_exp_tanh(aotk, oracle):
    """silu/gelu through the device expf/tanhf against glibc over a wide range."""
    rng = np.random.default_rng(3)
    h = np.concatenate([rng.standard_normal(100000) * 10, np.linspace(-100, 100, 100000),
                        [0.0, -0.0, 1e-30, -1e-30, 88.7, -104.0, 32.564632415771484, 63.1]]).astype(np.float32)
    up = np.ones_like(h)
    for fn, name in ((aotk.silu_mul, "or_silu_mul"), (aotk.gelu_mul, "or_gelu_mul")):
        ref = h.copy()
        getattr(oracle.load(), name)(oracle.ptr(ref), oracle.ptr(up), ref.size)
        got = fn(h, up)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), name


def _stress_rows(rng, n):
    rows = [rng.standard_normal(n), rng.standard_normal(n) * 1e-3, rng.standard_normal(n) * 50]
    t = np.where(rng.random(n) < 0.3, 2.0 ** -12, 1.0)  # squares 2^-24 next to 1.0: exact ties
    rows.append(t * rng.choice([1, -1], n))
    t = rng.integers(0, 4, n).astype(np.float64)
    t[: n // 8] = 0.0  # leading zeros
    rows.append(t)
    t = rng.standard_normal(n) * 1e-6
    t[n // 2] = 1e3  # a huge element mid-way
    rows.append(t)
    t = rng.standard_normal(n) * 1e3
    t[1:] *= 1e-9  # huge first element, then tiny ones
    rows.append(t)
    t = np.exp(rng.uniform(-20, 5, n)) * rng.choice([1, -1], n)  # wide dynamic range
    rows.append(t)
    rows.append(np.full(n, 3.0 * 2.0 ** -12))
    return np.array(rows, np.float32)


@pytest.mark.parametrize("n", [256, 2048, 2560, 4096, 8192])
def test_exact_sequential_sum_rmsnorm(aotk, oracle, n):
    """rmsnorm's sum of squares replays the reference's sequential order bit for bit."""
    rng = np.random.default_rng(n)
    x = _stress_rows(rng, n)
    w = np.ones(n, np.float32)
    got = aotk.rmsnorm(x, w, 1e-5)
    ref = np.stack([_or_rmsnorm(oracle, r, w) for r in x])
    bad = [i for i in range(len(x)) if not np.array_equal(got[i].view(np.uint32), ref[i].view(np.uint32))]
    assert not bad, f"rows {bad} differ"


@pytest.mark.parametrize("n", [2048, 2560, 4096])
def test_exact_sequential_sum_fuzz(aotk, oracle, n):
    """rmsnorm over 240 seeded rows of mixed scales, heavy tails, runs of
    equal values and sparse zeros (the sums' binade crossings and .5 ties
    fall at many different places): every row bit for bit."""
    rng = np.random.default_rng(1000 + n)
    rows = []
    for i in range(240):
        kind = i % 6
        if kind == 0:
            r = rng.standard_normal(n) * 10.0 ** rng.uniform(-4, 3)
        elif kind == 1:
            r = rng.standard_t(2, n)
        elif kind == 2:
            r = np.repeat(rng.standard_normal(n // 16), 16) * 2.0 ** rng.integers(-20, 10)
        elif kind == 3:
            r = np.where(rng.random(n) < 0.9, 0.0, rng.standard_normal(n))
        elif kind == 4:
            r = rng.integers(-8, 8, n) * 2.0 ** rng.integers(-12, 4)
        else:
            r = np.exp(rng.uniform(-15, 3, n)) * rng.choice([1, -1], n)
        rows.append(r)
    x = np.array(rows, np.float32)
    w = np.ones(n, np.float32)
    got = aotk.rmsnorm(x, w, 1e-5)
    ref = np.stack([_or_rmsnorm(oracle, r, w) for r in x])
    bad = [i for i in range(len(x)) if not np.array_equal(got[i].view(np.uint32), ref[i].view(np.uint32))]
    assert not bad, f"rows {bad[:10]} differ"


@pytest.mark.parametrize("n", [7, 64, 1000, 4096, 8192, 9000])
def test_exact_sequential_sum_softmax(aotk, oracle, n):
    rng = np.random.default_rng(n + 1)
    for s in (rng.standard_normal(n) * 4, rng.standard_normal(n) * 0.01, np.linspace(-30, 0, n),
              np.where(rng.random(n) < 0.5, 0.0, -16.635532)):
        s = s.astype(np.float32)
        ref = s.copy()
        oracle.load().or_softmax(oracle.ptr(ref), ref.size)
        assert np.array_equal(aotk.softmax(s).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("kind", [Q4_K, Q6_K, Q8_0, Q4_0, F16, F32], ids=lambda k: NAMES[k])
def test_fused_products(aotk, oracle, kind):
    """aotk_matvec3 / aotk_matvec2 / aotk_matmul2 (matvec.rs:321-439,
    :569-583): one launch over the concatenated rows, each output equal to
    its own product bit for bit."""
    rng = np.random.default_rng(90 + kind)
    cols = 1024
    shapes = [(96, cols), (32, cols), (40, cols)]
    raws = [weights(kind, r, c, 50 + i, oracle) for i, (r, c) in enumerate(shapes)]
    ws = [aotk.Weight(kind, raw, r, c) for raw, (r, c) in zip(raws, shapes)]
    x = rng.standard_normal(cols).astype(np.float32)
    act = oracle.quantize_act(kind, x)
    got = aotk.matvec3(ws, act)
    for g, raw, (r, c) in zip(got, raws, shapes):
        ref = oracle.matvec(kind, raw, act, r, c)
        assert np.array_equal(g.view(np.uint32), ref.view(np.uint32))
    ub = weights(kind, 96, cols, 77, oracle)
    wb = aotk.Weight(kind, ub, 96, cols)
    ga, gb = aotk.matvec2(ws[0], wb, act)
    assert np.array_equal(ga.view(np.uint32), oracle.matvec(kind, raws[0], act, 96, cols).view(np.uint32))
    assert np.array_equal(gb.view(np.uint32), oracle.matvec(kind, ub, act, 96, cols).view(np.uint32))
    for m in (5, 64):
        xs = np.concatenate([oracle.quantize_act(kind, rng.standard_normal(cols).astype(np.float32)) for _ in range(m)])
        ma, mb = aotk.matmul2(ws[0], wb, xs, m)
        assert np.array_equal(ma.view(np.uint32), oracle.matmul(kind, raws[0], xs, m, 96, cols).reshape(m, 96).view(np.uint32))
        assert np.array_equal(mb.view(np.uint32), oracle.matmul(kind, ub, xs, m, 96, cols).reshape(m, 96).view(np.uint32))
    with pytest.raises(aotk.AotkError, match="differ"):
        aotk.matvec2(ws[0], ws[1], act)
