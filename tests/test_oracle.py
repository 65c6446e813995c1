"""CPU tests: the oracle (C restatement of the reference's avx2+f16c path)
pinned against the reference's own test vectors, invariants and closed forms.

Each test names the reference test or fact it restates. The seeded
generators are restatements of the reference tests' own generators so the
same vectors are exercised:
  * quantize.rs:301-311  `data(n, seed)`: xorshift32 (13, 17, 5)
  * tests/dots.rs:10-21  `Rng`: xorshift64 (13, 7, 17), f() = (next % 20001) / 1e4 - 1
"""
import ctypes as C
import math
import struct

import numpy as np
import pytest

from oracle import oracle as O

F32, F16, BF16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K = range(9)  # quant.rs Kind order
KIND_NAMES = ["F32", "F16", "BF16", "Q4_0", "Q5_0", "Q8_0", "Q4_K", "Q5_K", "Q6_K"]


def f32(v):
    return float(np.float32(v))


class RefRng:
    """tests/dots.rs:10-21."""

    def __init__(self, seed):
        self.s = seed & 0xFFFFFFFFFFFFFFFF

    def next(self):
        M = 0xFFFFFFFFFFFFFFFF
        self.s ^= (self.s << 13) & M
        self.s ^= self.s >> 7
        self.s ^= (self.s << 17) & M
        return self.s

    def f(self):
        return f32(f32(self.next() % 20001) / f32(10000.0) - f32(1.0))

    def vec(self, n, scale=1.0):
        return np.array([f32(self.f() * f32(scale)) for _ in range(n)], np.float32)


def ref_data(n, seed):
    """quantize.rs:301-311 (u32 xorshift 13/17/5; s / u32::MAX * 2 - 1 in f32)."""
    M = 0xFFFFFFFF
    s = (seed * 2654435761 + 12345) & M
    out = np.empty(n, np.float32)
    umax = np.float32(4294967295.0)
    for i in range(n):
        s ^= (s << 13) & M
        s ^= s >> 17
        s ^= (s << 5) & M
        out[i] = np.float32(np.float32(s) / umax) * np.float32(2.0) - np.float32(1.0)
    return out


# ----------------------------------------------------------------- halves

def test_f16_known_values():
    """quant.rs:450-465 f16_roundtrip."""
    lib = O.load()
    for v in [0.0, 1.0, -1.0, 0.5, 65504.0, 1e-5, 6.1e-5, 1.2345, -0.333, 1e-7]:
        v = f32(v)
        back = lib.or_f16_to_f32(lib.or_f32_to_f16(v))
        assert abs(back - v) <= abs(v) * 1e-3 + 1e-7
    assert lib.or_f16_to_f32(0x3C00) == 1.0
    assert lib.or_f16_to_f32(0xC000) == -2.0
    assert lib.or_f16_to_f32(0x0001) == f32(5.9604645e-8)
    assert math.isinf(lib.or_f16_to_f32(0x7C00))
    assert math.isnan(lib.or_f16_to_f32(0x7E00))
    assert lib.or_f32_to_f16(1.0) == 0x3C00
    assert lib.or_f32_to_f16(float("inf")) == 0x7C00
    assert lib.or_f32_to_f16(f32(1e-8)) == 0


def test_f16_matches_ieee_everywhere():
    """IEEE binary16 (quant.rs:96-150 implements it): every half decodes like
    numpy's float16, and f32 -> f16 rounds to nearest even like numpy."""
    lib = O.load()
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([lib.or_f16_to_f32(int(v)) for v in h], np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()
    rng = np.random.default_rng(7)
    xs = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(100),
        (rng.standard_normal(5000) * 1e-5).astype(np.float32),  # subnormal halves
        np.array([65519.0, 65520.0, 6.1035156e-05, 2.9802322e-08, 2.9802326e-08, -0.0], np.float32),
    ])
    got = np.array([lib.or_f32_to_f16(float(v)) for v in xs], np.uint16)
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    assert (got == want).all()


def test_bf16_closed_form():
    """bf16 is the top half of an f32; encoding rounds to nearest even."""
    lib = O.load()
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 2**32, 5000, dtype=np.uint64).astype(np.uint32)
    xs = bits.view(np.float32)
    xs = xs[np.isfinite(xs)]
    for v in xs[:2000]:
        b = int(np.float32(v).view(np.uint32))
        up = b + 0x7FFF + ((b >> 16) & 1)
        assert lib.or_f32_to_bf16(float(v)) == (up >> 16) & 0xFFFF
    for h in range(0, 65536, 97):
        assert struct.unpack("<f", struct.pack("<I", h << 16))[0] == pytest.approx(lib.or_bf16_to_f32(h), nan_ok=True)


# ---------------------------------------------------- activation quantizers

def test_q8_0_activation():
    """quant.rs:467-479."""
    x = np.array([(i - 32.0) / 7.0 for i in range(64)], np.float32)
    out = O.quantize_q8_0(x)
    assert len(out) == 2
    for i, blk in enumerate(out):
        v = blk["qs"].astype(np.float32) * blk["d"]
        assert np.all(np.abs(v - x[i * 32:(i + 1) * 32]) < 0.05)


def test_q8_k_bsums():
    """quant.rs:481-490, and the same on random data of many blocks."""
    x = np.array([((i * 37) % 101) - 50.0 for i in range(256)], np.float32)
    blk = O.quantize_q8_k(x)[0]
    for j in range(16):
        assert int(blk["qs"][j * 16:(j + 1) * 16].astype(np.int32).sum()) == int(blk["bsums"][j])
    xs = np.random.default_rng(5).standard_normal(256 * 40).astype(np.float32)
    q = O.quantize_q8_k(xs)
    assert (q["qs"].astype(np.int32).reshape(40, 16, 16).sum(2) == q["bsums"]).all()


def test_q8_activation_invariants():
    """Both quantizers: |q| <= 127 with the largest |x| of a block at |q| =
    127, and q * d within d / 2 of x (round to nearest); an all-zero block
    quantizes to d = 0 (quant.rs:231-283)."""
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(256 * 8) * np.exp(rng.standard_normal(256 * 8))).astype(np.float32)
    x[256:512] = 0.0
    for q, bs in ((O.quantize_q8_k(x), 256), (O.quantize_q8_0(x), 32)):
        for i, blk in enumerate(q):
            xb = x[i * bs:(i + 1) * bs]
            qs = blk["qs"].astype(np.int32)
            if not xb.any():
                assert blk["d"] == 0.0 and not qs.any()
                continue
            assert np.abs(qs).max() == 127
            assert np.abs(qs).max() <= 127
            d = abs(float(blk["d"]))
            err = np.abs(qs * np.float64(blk["d"]) - xb)
            assert err.max() <= d * 0.5 + 1e-6 * np.abs(xb).max()


# --------------------------------------------------------- weight encoders

@pytest.mark.parametrize("kind,tol", [(F32, 1e-7), (F16, 1e-3), (BF16, 1e-2), (Q8_0, 1e-2), (Q4_0, 0.1),
                                      (Q5_0, 0.05), (Q4_K, 0.08), (Q5_K, 0.04), (Q6_K, 0.02)])
def test_encoder_roundtrip(kind, tol):
    """quantize.rs:313-333: encode 512 values of `data(512, kind + 1)`, decode,
    mean abs error below the reference's bound; row_bytes as quant.rs:20-87."""
    x = ref_data(512, kind + 1)
    enc = O.quantize_rows(kind, x[None, :])
    sizes = {F32: 2048, F16: 1024, BF16: 1024, Q8_0: 16 * 34, Q4_0: 16 * 18, Q5_0: 16 * 22, Q4_K: 2 * 144,
             Q5_K: 2 * 176, Q6_K: 2 * 210}
    assert enc.shape[1] == sizes[kind]
    dec = O.dequant_rows(kind, enc, 512)[0]
    assert float(np.abs(x - dec).mean()) < tol


def test_dequant_closed_forms():
    """Dequantization of hand-built blocks against the formulas of
    quant.rs:300-443 with values where every product is exact."""
    # Q8_0: d = 0.5 (f16 0x3800), qs = -16..15 -> q * d
    blk = struct.pack("<H", 0x3800) + bytes((np.arange(-16, 16) & 0xFF).astype(np.uint8))
    out = O.dequant_rows(Q8_0, np.frombuffer(blk, np.uint8), 32)[0]
    assert (out == np.arange(-16, 16) * 0.5).all()
    # Q4_0: d = 2, nibbles j and j+16 from byte j -> (q - 8) * d
    qs = np.arange(16, dtype=np.uint8) | (np.arange(15, -1, -1, dtype=np.uint8) << 4)
    blk = struct.pack("<H", 0x4000) + qs.tobytes()
    out = O.dequant_rows(Q4_0, np.frombuffer(blk, np.uint8), 32)[0]
    want = np.concatenate([np.arange(16) - 8, np.arange(15, -1, -1) - 8]) * 2.0
    assert (out == want).all()
    # Q5_0: high bit j of qh sets bit 4 of element j -> (q - 16) * d
    qh = 0xA5A5F00F
    blk = struct.pack("<HI", 0x3C00, qh) + qs.tobytes()
    out = O.dequant_rows(Q5_0, np.frombuffer(blk, np.uint8), 32)[0]
    hb = np.array([(qh >> j) & 1 for j in range(32)])
    want = np.concatenate([np.arange(16), np.arange(15, -1, -1)]) + 16 * hb - 16
    assert (out == want).all()
    # Q4_K: d = 1, dmin = 0.5, scales 1..8 / mins 0..7 (6-bit packing of
    # quant.rs:292-298 for j < 4 is plain bytes) -> (d*sc)*q - dmin*m
    sc = [1, 2, 3, 4]
    mn = [0, 1, 2, 3]
    scales = bytes(sc + mn + [0, 0, 0, 0])
    qsb = np.array([(i % 16) | (((i * 7) % 16) << 4) for i in range(128)], np.uint8)
    blk = struct.pack("<HH", 0x3C00, 0x3800) + scales + qsb.tobytes()
    out = O.dequant_rows(Q4_K, np.frombuffer(blk, np.uint8), 256)[0]
    for j in range(4):  # sub-blocks 0..3 use scale/min j (j < 4)
        for l in range(32):
            b = qsb[32 * (j // 2) + l]
            q = (b >> 4) if j % 2 else (b & 15)
            assert out[32 * j + l] == np.float32(sc[j]) * q - np.float32(0.5) * mn[j]
    # Q6_K: d = 0.25, scales i8 -> d*sc*(q-32)
    ql = np.arange(128, dtype=np.uint8)
    qh6 = np.full(64, 0b11100100, np.uint8)
    scs = np.array([1, -2, 3, -4, 5, -6, 7, -8, 2, 2, 2, 2, -1, -1, -1, -1], np.int8)
    blk = ql.tobytes() + qh6.tobytes() + scs.tobytes() + struct.pack("<H", 0x3400)
    out = O.dequant_rows(Q6_K, np.frombuffer(blk, np.uint8), 256)[0]
    for n in range(2):
        for l in range(32):
            for quarter in range(4):
                lo = ql[64 * n + l + 32 * (quarter & 1)]
                lo = (lo >> 4) if quarter >= 2 else (lo & 15)
                q = int(lo) | (((int(qh6[32 * n + l]) >> (2 * quarter)) & 3) << 4)
                idx = 128 * n + 32 * quarter + l
                s = int(scs[8 * n + l // 16 + 2 * quarter])
                assert out[idx] == np.float32(np.float32(0.25) * s) * np.float32(q - 32)


# --------------------------------------------------------------------- dots

def dot_case(kind, cols, seed):
    """tests/dots.rs:52-89 check_kind: weights rng.f(), x rng.f() * 3."""
    rng = RefRng(seed)
    w = rng.vec(cols)
    x = rng.vec(cols, 3.0)
    wq = O.quantize_rows(kind, w[None, :])[0]
    xa = O.quantize_act(kind, x)
    return w, x, wq, xa


@pytest.mark.parametrize("kind,cols,seed", [
    (Q4_0, 32, 1), (Q4_0, 64, 2), (Q4_0, 96, 3), (Q4_0, 2048, 4), (Q4_0, 5632, 5),
    (Q5_0, 32, 11), (Q5_0, 64, 12), (Q5_0, 96, 13), (Q5_0, 2048, 14),
    (Q8_0, 32, 11), (Q8_0, 64, 12), (Q8_0, 96, 13), (Q8_0, 2048, 14),
    (Q4_K, 256, 21), (Q4_K, 512, 22), (Q4_K, 2048, 23), (Q4_K, 5632, 24),
    (Q5_K, 256, 31), (Q5_K, 512, 32), (Q5_K, 2048, 33),
    (Q6_K, 256, 41), (Q6_K, 512, 42), (Q6_K, 2048, 43), (Q6_K, 8192, 44),
    (F16, 8, 51), (F16, 12, 52), (F16, 64, 53), (F16, 2048, 54), (F16, 2053, 55),
    (BF16, 8, 51), (BF16, 2053, 55), (F32, 12, 52), (F32, 2053, 55),
])
def test_dots_against_float_and_scalar(kind, cols, seed):
    """tests/dots.rs:52-89: every kernel set within 0.02 * sum|x| of the
    float reference of the dequantized row; avx2 within 1e-4 rel of scalar;
    K-quant avx2 == scalar bit for bit (exact integer sums, same fold)."""
    w, x, wq, xa = dot_case(kind, cols, seed)
    deq = O.dequant_rows(kind, wq, cols)[0]
    fref = float(np.dot(deq.astype(np.float64), x.astype(np.float64)))
    scale = float(np.abs(x).sum()) * 0.02 + 1e-3
    s = O.dot(kind, wq, xa, cols, "scalar")
    a = O.dot(kind, wq, xa, cols, "avx2")
    assert abs(s - fref) < scale and abs(a - fref) < scale
    assert abs(a - s) <= abs(s) * 1e-4 + 1e-3
    if kind in (Q4_K, Q5_K, Q6_K):
        assert np.float32(a).view(np.uint32) == np.float32(s).view(np.uint32)


def test_kquant_dot_is_exact_integer_fold():
    """Brute force: with an activation whose Q8_K scale is a power of two and a
    weight row with f16 scales d = 1, dmin = 0, the K-quant dot equals the
    exact dot of the dequantized row with the de-quantized activation (every
    product and partial sum is an integer below 2^24)."""
    rng = np.random.default_rng(2)
    for kind in (Q4_K, Q5_K, Q6_K):
        cols = 1024
        # activation: integers in [-127, 127] with one -127 per block; the
        # signed max is -127, so iscale = 1 and d = 1
        y = rng.integers(-100, 101, cols).astype(np.float32)
        y[::256] = -127.0
        xa = O.quantize_q8_k(y)
        assert (xa["d"] == 1.0).all() and (xa["qs"].reshape(-1) == y).all()
        w = O.quantize_rows(kind, (rng.standard_normal((1, cols)) * 0.02).astype(np.float32))[0].copy()
        tsz = {Q4_K: 144, Q5_K: 176, Q6_K: 210}[kind]
        for b in range(cols // 256):
            blk = w[b * tsz:(b + 1) * tsz]
            if kind == Q6_K:
                blk[208:210] = np.frombuffer(struct.pack("<H", 0x3C00), np.uint8)
            else:
                blk[0:4] = np.frombuffer(struct.pack("<HH", 0x3C00, 0x0000), np.uint8)
        deq = O.dequant_rows(kind, w, cols)[0].astype(np.float64)
        exact = float(np.dot(deq, y.astype(np.float64)))
        assert abs(exact) < 2**24
        for k in ("scalar", "avx2"):
            assert O.dot(kind, w, xa, cols, k) == exact


def test_x4_matches_single():
    """tests/dots.rs:159-203 (seed 777): 1x4 micro-kernels bit-identical."""
    lib = O.load()
    rng = RefRng(777)
    cols = 2048
    for kind in (Q4_0, Q5_0, Q8_0, Q4_K, Q6_K):
        w = rng.vec(cols)
        wq = np.ascontiguousarray(O.quantize_rows(kind, w[None, :])[0])
        xs = [O.quantize_act(kind, rng.vec(cols, 2.0)) for _ in range(4)]
        ptrs = (C.c_void_p * 4)(*[x.ctypes.data for x in xs])
        out = (C.c_float * 4)()
        assert lib.or_dot_avx2_x4(kind, O.ptr(wq), ptrs, cols, out) == 0
        for i in range(4):
            single = O.dot(kind, wq, xs[i], cols, "avx2")
            assert np.float32(out[i]).view(np.uint32) == np.float32(single).view(np.uint32)


def test_matmul_matches_matvec_bitwise():
    """tests/dots.rs:205-266 (seed 4242, rows 37, cols 512, m 1/3/4/7/9)."""
    rng = RefRng(4242)
    rows, cols = 37, 512
    pool = O.Pool(3)
    for kind in (Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K, F16):
        w = np.stack([rng.vec(cols) for _ in range(rows)])
        wq = O.quantize_rows(kind, w)
        for m in (1, 3, 4, 7, 9):
            xs = rng.vec(m * cols)
            xa = O.quantize_act(kind, xs)
            batched = O.matmul(kind, wq, xa, m, rows, cols, pool)
            per = len(xa) // m
            for i in range(m):
                single = O.matvec(kind, wq, xa[i * per:(i + 1) * per], rows, cols, pool)
                assert (single.view(np.uint32) == batched[i * rows:(i + 1) * rows].view(np.uint32)).all()


def test_matvec_parallel_matches_serial():
    """tests/dots.rs:135-157 (seed 99): 1 vs 4 threads bit-identical, each row
    within 0.5 of the float reference."""
    rng = RefRng(99)
    rows, cols = 37, 512
    w = np.stack([rng.vec(cols) for _ in range(rows)])
    x = rng.vec(cols)
    wq = O.quantize_rows(Q4_K, w)
    xa = O.quantize_q8_k(x)
    o1 = O.matvec(Q4_K, wq, xa, rows, cols, O.Pool(1))
    o4 = O.matvec(Q4_K, wq, xa, rows, cols, O.Pool(4))
    assert (o1.view(np.uint32) == o4.view(np.uint32)).all()
    deq = O.dequant_rows(Q4_K, wq, cols).astype(np.float64)
    assert np.all(np.abs(o1 - deq @ x.astype(np.float64)) < 0.5)


# ---------------------------------------------------------------------- ops

def arr(v):
    return np.ascontiguousarray(np.array(v, np.float32))


def test_softmax_sums_to_one():
    """ops.rs:224-230."""
    v = arr([1.0, 2.0, 3.0, -1.0])
    O.load().or_softmax(O.ptr(v), 4)
    assert abs(float(v.sum()) - 1.0) < 1e-6
    assert v[2] > v[1] > v[0] > v[3]


def test_rmsnorm_unit_weights():
    """ops.rs:232-241."""
    x, w, out = arr([3.0, 4.0]), arr([1.0, 1.0]), arr([0.0, 0.0])
    O.load().or_rmsnorm(O.ptr(out), O.ptr(x), O.ptr(w), 2, 0.0)
    rms = math.sqrt(12.5)
    assert abs(out[0] - 3.0 / rms) < 1e-6 and abs(out[1] - 4.0 / rms) < 1e-6


def test_rope_rotates_pairs():
    """ops.rs:243-254 and :256-277 (NEOX pairs, permutation equivalence)."""
    lib = O.load()
    inv, cs = arr([1.0, 0.5]), arr([0.0] * 4)
    lib.or_rope_cos_sin(O.ptr(cs), O.ptr(inv), 2, math.pi / 2)
    x = arr([1.0, 0.0, 1.0, 0.0])
    lib.or_rope(O.ptr(x), 1, 4, 4, O.ptr(cs), 0)
    r = 1 / math.sqrt(2)
    assert abs(x[0]) < 1e-6 and abs(x[1] - 1) < 1e-6 and abs(x[2] - r) < 1e-6 and abs(x[3] - r) < 1e-6
    x = arr([1.0, 1.0, 0.0, 0.0])
    lib.or_rope(O.ptr(x), 1, 4, 4, O.ptr(cs), 1)
    assert abs(x[0]) < 1e-6 and abs(x[2] - 1) < 1e-6 and abs(x[1] - r) < 1e-6 and abs(x[3] - r) < 1e-6
    inv8, cs8 = arr([1.0, 0.7, 0.4, 0.1]), arr([0.0] * 8)
    lib.or_rope_cos_sin(O.ptr(cs8), O.ptr(inv8), 4, 3.0)
    src = arr([i * 0.37 - 1.0 for i in range(8)])
    neox = src.copy()
    lib.or_rope(O.ptr(neox), 1, 8, 8, O.ptr(cs8), 1)
    perm = arr([v for i in range(4) for v in (src[i], src[i + 4])])
    lib.or_rope(O.ptr(perm), 1, 8, 8, O.ptr(cs8), 0)
    for i in range(4):
        assert abs(neox[i] - perm[2 * i]) < 1e-6 and abs(neox[i + 4] - perm[2 * i + 1]) < 1e-6


def test_rmsnorm_heads():
    """ops.rs:279-293."""
    w, x = arr([2.0, 1.0]), arr([3.0, 4.0, 0.5, 0.5])
    O.load().or_rmsnorm_heads(O.ptr(x), O.ptr(w), 2, 2, 0.0)
    rms0, rms1 = math.sqrt(12.5), 0.5
    assert abs(x[0] - 6 / rms0) < 1e-5 and abs(x[1] - 4 / rms0) < 1e-5
    assert abs(x[2] - 1 / rms1) < 1e-5 and abs(x[3] - 0.5 / rms1) < 1e-5


def attention(q, kc, vc, n_head, n_kv, hd, ctx, layer, pos, window, n_threads=2):
    out = np.zeros(n_head * hd, np.float32)
    pool = O.Pool(n_threads)
    O.load().or_attention(pool.p, O.ptr(out), O.ptr(q), O.ptr(kc), O.ptr(vc), n_head, n_kv, hd, ctx, layer, pos,
                          1, window)
    return out


def test_attention_closed_forms():
    """ops.rs:295-344: one position returns its value; window 1 sees only the
    newest position; equal keys average the values."""
    q = np.ones(8, np.float32)
    kc = np.zeros(16, np.float32)
    vc = np.zeros(16, np.float32)
    kc[0:4] = [1, 2, 3, 4]
    vc[0:4] = [5, 6, 7, 8]
    out = attention(q, kc, vc, 2, 1, 4, 4, 0, 0, 0)
    assert list(out[:4]) == [5, 6, 7, 8] and list(out[4:]) == [5, 6, 7, 8]
    kc[4:8] = [1, 2, 3, 4]
    vc[4:8] = [1, 1, 1, 1]
    assert list(attention(q, kc, vc, 2, 1, 4, 4, 0, 1, 1)[:4]) == [1, 1, 1, 1]
    two = attention(q, kc, vc, 2, 1, 4, 4, 0, 1, 2)
    assert list(two[:4]) == [3.0, 3.5, 4.0, 4.5]
    assert (two == attention(q, kc, vc, 2, 1, 4, 4, 0, 1, 0)).all()


def test_gelu_values():
    """ops.rs:346-353."""
    lib = O.load()
    assert abs(lib.or_gelu(0.0)) < 1e-7
    assert abs(lib.or_gelu(1.0) - 0.841192) < 1e-5
    assert abs(lib.or_gelu(-1.0) + 0.158808) < 1e-5
    h, up = arr([1.0, -1.0]), arr([2.0, 2.0])
    lib.or_gelu_mul(O.ptr(h), O.ptr(up), 2)
    assert abs(h[0] - 1.682384) < 1e-5 and abs(h[1] + 0.317616) < 1e-5


def test_silu_closed_form():
    """ops.rs:115-120: v / (1 + exp(-v)) * up, silu(0) = 0, large v -> v."""
    h, up = arr([0.0, 20.0, -20.0, 1.0]), arr([3.0, 1.0, 1.0, 1.0])
    O.load().or_silu_mul(O.ptr(h), O.ptr(up), 4)
    assert h[0] == 0.0 and abs(h[1] - 20.0) < 1e-5 and abs(h[2]) < 1e-7
    assert abs(h[3] - 1 / (1 + math.exp(-1))) < 1e-6


def test_argmax_first_index():
    """sampler.rs:99-109: first index of the strict max; NaN never wins."""
    assert O.argmax(arr([1.0, 3.0, 3.0, 2.0])) == 1
    assert O.argmax(arr([float("nan"), 1.0, 0.5])) == 1
    assert O.argmax(arr([-float("inf"), -1.0])) == 1


def test_window_start():
    """ops.rs:171-177."""
    lib = O.load()
    assert lib.or_window_start(5, 0) == 0
    assert lib.or_window_start(5, 2) == 4
    assert lib.or_window_start(1, 4) == 0


def test_inv_freq_closed_form():
    """state.rs:304-319: base^(-2i/rot_dim)."""
    out = np.zeros(64, np.float32)
    O.load().or_inv_freq(O.ptr(out), 128, 500000.0, None)
    want = 500000.0 ** (-np.arange(64) * 2.0 / 128)
    assert np.allclose(out, want, rtol=2e-6)
