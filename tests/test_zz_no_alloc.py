"""aotk_matmul_noalloc (the entry point that allocates nothing) against
aotk_matmul, through the C ABI: bit for bit, two calls in a row with the
second smaller, every activation format, and the size limit."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q6_K, F16 = 5, 6, 8, 1


def _weights(oracle, kind, rows, cols, seed):
    rng = np.random.default_rng(seed)
    return oracle.quantize_rows(kind, (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32))


@pytest.mark.parametrize("kind", [Q4_K, Q6_K, Q8_0, F16])
def test_noalloc_matches_matmul(aotk, oracle, kind):
    rng = np.random.default_rng(40 + kind)
    cols, rows = 4096, 1100
    raw = _weights(oracle, kind, rows, cols, kind)
    w = aotk.Weight(kind, raw, rows, cols)
    for m in (64, 5):  # the second call is smaller: stale staging must not leak in
        xs = rng.standard_normal((m, cols)).astype(np.float32)
        acts = np.concatenate([oracle.quantize_act(kind, x) for x in xs])
        want = aotk.matmul(w, acts, m)
        got = aotk.matmul_noalloc(w, acts, m)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (kind, m)
        ref = oracle.matmul(kind, raw, acts, m, rows, cols).reshape(m, rows)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (kind, m)
    w.free()


def test_noalloc_rejects_oversize(aotk, oracle):
    cols, rows, m = 65536, 4, 64  # 64 x 65536 Q8_K inputs need ~4.7 MiB of staging
    raw = _weights(oracle, Q4_K, rows, cols, 1)
    w = aotk.Weight(Q4_K, raw, rows, cols)
    acts = np.zeros(m * (cols // 256), oracle.Q8_K_DTYPE)
    with pytest.raises(aotk.AotkError, match="staging bytes"):
        aotk.matmul_noalloc(w, acts, m)
    w.free()
