"""CPU tests of the host side: the C-ABI library loads and exports every
entry point the header declares, the config tensor tables have the sizes the
reference's model shapes imply, and the product path fails loudly without a
GPU (no CPU fallback)."""
import ctypes as C
import os
import re

import pytest

from aotk import abi, configs

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "aotk.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(aotk_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_function():
    lib = abi.load()
    names = header_functions()
    assert len(names) > 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_block_layouts_match_header():
    """aotk_block_q8_0 / q8_k are the reference's BlockQ8_0 (36 B incl. f32 d)
    and BlockQ8_K (292 B) (quant.rs:186-229)."""
    from oracle import oracle as O
    assert O.Q8_0_DTYPE.itemsize == 36 and O.Q8_K_DTYPE.itemsize == 292
    text = open(HEADER).read()
    assert "aotk_block_q8_0" in text and "aotk_block_q8_k" in text


@pytest.mark.parametrize("kind,cols,want", [
    (abi.F32, 512, 2048), (abi.F16, 512, 1024), (abi.BF16, 512, 1024), (abi.Q4_0, 512, 288),
    (abi.Q5_0, 512, 352), (abi.Q8_0, 512, 544), (abi.Q4_K, 512, 288), (abi.Q5_K, 512, 352),
    (abi.Q6_K, 5632, 22 * 210)])
def test_row_bytes(kind, cols, want):
    """quant.rs:20-87 sizes, computed by the library's host code."""
    assert abi.row_bytes(kind, cols) == want
    assert abi.load().aotk_row_bytes(kind, cols) == want


@pytest.mark.parametrize("name,mb", [("tinyllama-1.1b-q4km", 667.5), ("llama3-8b-q4km", 4877.0)])
def test_decode_weight_bytes(name, mb):
    """Weight bytes per decode token of the configs (TinyLlama 27.90 MB/layer +
    53.8 MB lm-head; Llama-3-8B 4.877 GB) from their Q4_K_M tensor tables."""
    spec = configs.build(name)
    assert abs(spec.decode_weight_bytes() / 1e6 - mb) / mb < 2e-3


def test_config_tables_are_aligned_and_disjoint():
    """Tensor data offsets 32-byte aligned like GGUF's tensor-data section, no
    overlap, and every tensor's length is rows * row_bytes(kind, cols)."""
    for name in configs.CONFIGS:
        spec = configs.build(name)
        ts = []
        s = spec.spec
        for t in [s.token_embd, s.output_norm, s.output] + [getattr(L, f) for L in spec.layers for f, _ in
                                                            type(L)._fields_ if f not in ("local_attn",)]:
            if isinstance(t, abi.Tensor) and t.kind != abi.NONE:
                ts.append(t)
        ts.sort(key=lambda t: t.off)
        end = 0
        for t in ts:
            assert t.off % 32 == 0 and t.off >= end
            assert t.len == t.rows * abi.row_bytes(t.kind, t.cols)
            end = t.off + t.len
        assert end <= spec.blob_len


def test_prompt_tokens_deterministic():
    a = configs.prompt_tokens(1, 64, 128256)
    assert a == configs.prompt_tokens(1, 64, 128256)
    assert all(0 <= t < 128256 for t in a) and len(set(a)) > 60


def test_init_fails_loudly_without_gpu():
    """No CPU fallback: without a visible GPU the library reports an error
    instead of computing anything."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    lib = abi.load()
    assert lib.aotk_init(0) == -1
    assert lib.aotk_last_error()
