"""Writes the golden fixtures of tests/golden/ from the CPU oracle.

The reference is Rust and cannot run here, so these vectors are produced by
the oracle (the C restatement of the reference's avx2+f16c kernels) after the
oracle itself is pinned by tests/test_oracle.py (the reference's own test
vectors, invariants and closed forms). They freeze the oracle's outputs so
that the GPU path and later oracle changes are checked against fixed data.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "aot-llm_amd")]

from oracle import oracle as O  # noqa: E402
from aotk import configs  # noqa: E402

KINDS = {"F32": 0, "F16": 1, "BF16": 2, "Q4_0": 3, "Q5_0": 4, "Q8_0": 5, "Q4_K": 6, "Q5_K": 7, "Q6_K": 8}


def matvec_fixture():
    """Per kind: 3 rows x 512 cols of N(0, 0.02) weights (seed 0x5EED), x N(0, 1),
    the encoded rows, the activation and the avx2 matvec output."""
    out = {}
    rng = np.random.default_rng(0x5EED)
    for name, kind in KINDS.items():
        w = (rng.standard_normal((3, 512)) * 0.02).astype(np.float32)
        x = rng.standard_normal(512).astype(np.float32)
        wq = O.quantize_rows(kind, w)
        xa = O.quantize_act(kind, x)
        y = O.matvec(kind, wq, xa, 3, 512, O.Pool(1))
        out[f"{name}_w"] = wq
        out[f"{name}_x"] = x
        out[f"{name}_xq"] = np.frombuffer(xa.tobytes(), np.uint8) if xa.dtype.names else np.zeros(0, np.uint8)
        out[f"{name}_deq"] = O.dequant_rows(kind, wq, 512)
        out[f"{name}_y"] = y
    return out


def model_fixture(name):
    """Tiny config: 6-token prompt, logits after it, 16 greedy tokens."""
    spec = configs.build(name)
    blob = O.synth_blob(spec, 0x5EED)
    toks = configs.prompt_tokens(1, 6, spec.d["vocab"])
    m = O.Model(spec, blob, 32, max_batch=8, n_threads=4)
    m.prompt(toks, batch=8)
    logits = m.logits()
    gen = m.generate(6, 16)
    m.close()
    return {"prompt": np.array(toks, np.uint32), "logits": logits, "greedy": np.array(gen, np.uint32)}


def main():
    O.load()
    np.savez_compressed(os.path.join(HERE, "matvec_512.npz"), **matvec_fixture())
    for name in ("tiny-llama", "tiny-q4km", "tiny-q8_0", "tiny-q5km"):
        np.savez_compressed(os.path.join(HERE, f"model_{name}.npz"), **model_fixture(name))
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main()
