"""Writes the full-length greedy-stream fixtures of the five benchmark configs
(tests/golden/stream_<config>.npz) from the CPU oracle.

Each config runs exactly as its benchmark line is written: the seeded
synthetic model (seed 0x5EED, the same bytes the device synthesises), a
random-id prompt (splitmix64 stream of seed 1 for the main workloads, seed 2
for the long-context prefills, as bench.py uses them) pushed through the
batched prompt loop (crates/aot-kernels/src/app.rs:474-485, chunks of 64),
then the greedy loop (app.rs:553-610):

    tinyllama-1.1b-q4km   6-token prompt,    32 greedy tokens   (configs[0])
    llama3-8b-q4km      512-token prompt,   128 greedy tokens   (configs[2])
    qwen3-8b-q8_0      4096-token prefill,  256 greedy tokens   (configs[3])
    gemma3-4b-q5km     8192-token prefill,  256 greedy tokens   (configs[4])

Stored per config: the prompt ids, the greedy stream, and for the prompt-end
and the last decode step's logits their SHA-256 (bit-exact check) plus the 16
largest values with their ids (diagnostics). The oracle is pinned by
tests/test_oracle.py and tests/test_oracle_forward.py; these fixtures freeze
its outputs at lengths the GPU tests cannot afford to recompute on the CPU.

    python tests/golden/make_streams.py [config ...]
    python tests/golden/make_streams.py --sampled [config ...]   (sampled_<config>.npz)
"""
import hashlib
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "aot-llm_amd")]

from oracle import oracle as O  # noqa: E402
from aotk import configs  # noqa: E402

SEED = 0x5EED
CHUNK = 64
# name: (prompt seed, prompt tokens, greedy tokens)
STREAMS = {
    "tinyllama-1.1b-q4km": (1, 6, 32),
    "llama3-8b-q4km": (1, 512, 128),
    "qwen3-8b-q8_0": (2, 4096, 256),
    "gemma3-4b-q5km": (2, 8192, 256),
}


def digest(logits):
    return np.frombuffer(hashlib.sha256(np.ascontiguousarray(logits, np.float32).tobytes()).digest(), np.uint8)


def top16(logits):
    idx = np.argsort(-logits, kind="stable")[:16].astype(np.uint32)
    return idx, logits[idx].astype(np.float32)


def stream(name, threads):
    pseed, n_prompt, n_gen = STREAMS[name]
    spec = configs.build(name)
    t0 = time.perf_counter()
    blob = O.synth_blob(spec, SEED, n_threads=threads)
    toks = configs.prompt_tokens(pseed, n_prompt, spec.d["vocab"])
    m = O.Model(spec, blob, n_prompt + n_gen, max_batch=CHUNK, n_threads=threads)
    m.prompt(toks, batch=CHUNK)
    lp = m.logits()
    t1 = time.perf_counter()
    gen = m.generate(n_prompt, n_gen)
    lf = m.logits()
    t2 = time.perf_counter()
    m.close()
    pi, pv = top16(lp)
    fi, fv = top16(lf)
    print(f"{name}: prompt {n_prompt} in {t1 - t0:.0f} s, {n_gen} greedy in {t2 - t1:.0f} s; head {gen[:8]}", flush=True)
    return dict(prompt=np.array(toks, np.uint32), greedy=np.array(gen, np.uint32), chunk=np.uint32(CHUNK),
                prompt_sha256=digest(lp), prompt_top_ids=pi, prompt_top_vals=pv,
                final_sha256=digest(lf), final_top_ids=fi, final_top_vals=fv)


# Sampled streams (the app.rs:553-610 loop with sampler.rs): every config
# of STREAMS at its written length with --temp 0.8 --top-k 40 --top-p 0.95
# --repeat-penalty 1.1 (window 64) and seed 42, the penalty window running
# over the prompt and the generated tokens
SAMPLED = {"tinyllama-1.1b-q4km": (1, 6, 32), "llama3-8b-q4km": (1, 512, 128),
           "qwen3-8b-q8_0": (2, 4096, 256), "gemma3-4b-q5km": (2, 8192, 256)}
SAMPLER = dict(temperature=0.8, top_k=40, top_p=0.95, repeat_penalty=1.1, repeat_last_n=64, seed=42)


def sampled(name, threads):
    pseed, n_prompt, n_gen = SAMPLED[name]
    spec = configs.build(name)
    blob = O.synth_blob(spec, SEED, n_threads=threads)
    toks = configs.prompt_tokens(pseed, n_prompt, spec.d["vocab"])
    m = O.Model(spec, blob, n_prompt + n_gen, max_batch=CHUNK, n_threads=threads)
    m.prompt(toks, batch=CHUNK)
    gen = m.generate_sampled(n_prompt, n_gen, O.Sampler(**SAMPLER), toks)
    m.close()
    print(f"{name} sampled: head {gen[:8]}", flush=True)
    return dict(prompt=np.array(toks, np.uint32), sampled=np.array(gen, np.uint32), chunk=np.uint32(CHUNK),
                **{k: np.float64(v) for k, v in SAMPLER.items()})


def main():
    O.load()
    args = sys.argv[1:]
    threads = min(os.cpu_count() or 1, 8)
    if args[:1] == ["--sampled"]:
        for name in args[1:] or list(SAMPLED):
            np.savez_compressed(os.path.join(HERE, f"sampled_{name}.npz"), **sampled(name, threads))
        return
    for name in args or list(STREAMS):
        np.savez_compressed(os.path.join(HERE, f"stream_{name}.npz"), **stream(name, threads))


if __name__ == "__main__":
    main()
