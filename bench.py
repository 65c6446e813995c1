#!/usr/bin/env python3
"""Benchmark of the MI355X aot-llm hot path (one GPU).

Workload: Llama-3-8B shape, Q4_K_M random-init
weights, a 512-token random-id prompt in 64-token chunks, then greedy decode.
A "step" is one decode token (one pass of the emitted forward() over the
model, batch 1). `value` = decode tok/s measured like the reference's stats
line (crates/aot-kernels/src/app.rs:642-660: forwards / generation seconds),
weights and KV cache resident in HBM.

Also reported on the same JSON line:
  prompt_tok_s   evaluated prompt tokens / prompt seconds (app.rs:651)
  prompt_int8_TOPs / prompt_int8_frac
                 the prompt's matmul work (2 x tokens x layer weights, 0.893
                 TOP per 64-token chunk) per second, and against the MI355X
                 dense int8 MFMA peak (5 POP/s)
  q4k_matvec     the Q4_K matvec kernel alone at the microbench shapes
                 (configs[1]), GB/s of algorithmic bytes, copies rotated past
                 the 256 MB Infinity Cache
  matvec_kinds   the same for the other seven kinds at every shape
  roofline       the dominant decode kernel (Q4_K matvec, 14336x4096) vs
                 MI355X HBM peak, timed with HIP events on the library stream
  prompt_hbm_frac
                 the prompt's binding roof at 64-token chunks: every chunk
                 streams the layer weights once, bytes / prompt time / 8 TB/s
  decode_hbm_frac
                 (weights + attended KV rows) per token x tok/s / 8 TB/s
  hbm_ceiling    this box's measured streaming ceilings (read-only probe at
                 the matvec's 33 MB and at 1 GiB, a 256 MiB copy kernel)
  other_configs  TinyLlama-1.1B Q4_K_M (configs[0]: 6-token prompt, 32
                 greedy tokens), Qwen3-8B Q8_0 (4096-token prefill, then 256
                 decode tokens) and Gemma-3-4B Q5_K_M (8192-token prefill,
                 then 256 decode tokens), each with HBM fractions
  cpu_baseline   the CPU oracle (restated avx2+f16c reference kernels) on a
                 bounded sample of the same workload on this host's cores,
                 plus the configs[1] matvec cells and bounded decode samples
                 of the Qwen3 / Gemma-3 configs on the host

  python bench.py [--gpus 1] [--steps 128] [--warmup 8] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "aot-llm_amd")]

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA
SEED = 0x5EED


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def matvec_bytes(kind, rows, cols):
    from aotk import abi
    return rows * abi.row_bytes(kind, cols) + abi.act_bytes(kind, cols) + 4 * rows


def layer_weight_bytes(spec):
    """Bytes of every layer matrix (what one prompt chunk streams once)."""
    return sum(getattr(spec.layers[i], n).len for i in range(spec.d["n_layer"])
               for n in ("wq", "wk", "wv", "wo", "gate", "up", "down"))


def kv_bytes_per_token(spec, first, n):
    """Mean KV-cache bytes one decode step reads (K and V rows of every
    attended position, f32) over decode positions first..first+n-1; local
    layers of a sliding-window model attend min(pos + 1, window) positions
    (window_start, crates/aot-kernels/src/ops.rs:171-177)."""
    d = spec.d
    kv_row = 2 * d["n_kv_head"] * d["head_dim"] * 4
    win = int(spec.spec.dims.swa_window)
    total = 0
    for li in range(d["n_layer"]):
        local = spec.layers[li].local_attn and win > 0
        for p in range(first, first + n):
            total += (min(p + 1, win) if local else p + 1) * kv_row
    return total / max(n, 1)


def hbm_ceiling(aotk):
    """The box's own streaming ceilings beside the 8 TB/s spec: a read-only
    probe over the Q4_K 14336x4096 matvec's 33 MB (rotated past 1 GB, the
    matvec's own launch size) and over 1 GiB, and a copy kernel over 256 MiB
    (read + write counted)."""
    out = {}
    small = 33_030_144  # 14336 x 4096 Q4_K weight bytes, rounded to 16
    shapes = (1, 2, 4, 8)  # 16-byte loads in flight per lane; the best one is the ceiling
    bufs = [aotk.DeviceBuffer(small) for _ in range(32)]
    ms = min(aotk.time_hbm(bufs, small, 320, loads_per_lane=u) for u in shapes)
    out["read_33MB_GBs"] = round(small / (ms * 1e-3) / 1e9, 1)
    out["read_33MB_us"] = round(ms * 1e3, 2)
    for b in bufs:
        b.free()
    big = 1 << 30
    bufs = [aotk.DeviceBuffer(big) for _ in range(2)]
    ms = min(aotk.time_hbm(bufs, big, 20, loads_per_lane=u) for u in shapes)
    out["read_1GiB_GBs"] = round(big / (ms * 1e-3) / 1e9, 1)
    q = 256 << 20
    ms = min(aotk.time_hbm(bufs, q, 20, copy=True, loads_per_lane=u) for u in shapes)
    out["copy_256MiB_GBs"] = round(2 * q / (ms * 1e-3) / 1e9, 1)
    for b in bufs:
        b.free()
    out["peak_GBs"] = HBM_PEAK_GBS
    out["note"] = ("k_hbm_read / k_hbm_copy (aotk_time_hbm): coalesced 16-byte loads, the best of 1/2/4/8 in flight "
                   "per lane, HIP events; copy GB/s counts read + written bytes")
    return out


def cpu_matvec_cells(aotk, shapes, kinds, budget_s=0.25):
    """configs[1] on the host: the oracle's avx2 matvec (matvec.rs:358-401
    drivers) for every kind and shape, the same 512 distinct device-encoded
    rows tiled to the full shape as the GPU cells, min(cores, 8) threads;
    GB/s of the same algorithmic bytes."""
    import numpy as np
    from oracle import oracle as O
    from aotk import abi
    threads = min(os.cpu_count() or 1, 8)
    pool = O.Pool(threads)
    out = {}
    for kind in kinds:
        cells = {}
        for rows, cols in shapes:
            rng = np.random.default_rng(1)
            base = aotk.quantize_rows(kind, (rng.standard_normal((min(rows, 512), cols)) * 0.02).astype(np.float32))
            w = np.resize(base, (rows, base.shape[1]))
            xa = O.quantize_act(kind, rng.standard_normal(cols).astype(np.float32))
            O.matvec(kind, w, xa, rows, cols, pool)  # warm-up (page-in)
            n, t = 0, time.perf_counter()
            while n < 2 or time.perf_counter() - t < budget_s:
                O.matvec(kind, w, xa, rows, cols, pool)
                n += 1
            dt = (time.perf_counter() - t) / n
            cells[f"{rows}x{cols}"] = round(matvec_bytes(kind, rows, cols) / dt / 1e9, 2)
            del w
        out[abi.KIND_NAMES[kind]] = cells
    return dict(GBs=out, threads=threads, kind="port", note="oracle avx2+f16c matvec per call, GB/s of the algorithmic bytes")


def cpu_decode_from_gpu_kv(spec, blob, st, n_ctx, first_tok, budget_s):
    """A bounded CPU sample of a long-context decode: the GPU's prefilled KV
    rows (bit-identical to the oracle's prefill, which the stream tests pin)
    copied into the oracle, then greedy decode forwards from n_ctx on
    min(cores, 8) threads until the budget is spent."""
    import numpy as np
    from oracle import oracle as O
    d = spec.d
    kvd = d["n_kv_head"] * d["head_dim"]
    threads = min(os.cpu_count() or 1, 8)
    ctx = n_ctx + 64
    k, v = st.kv_download(n_ctx)
    m = O.Model(spec, blob, ctx, max_batch=1, n_threads=threads, kernels=1)
    rk, rv = m.kv(ctx)
    rk.reshape(d["n_layer"], ctx, kvd)[:, :n_ctx] = k.reshape(d["n_layer"], n_ctx, kvd)
    rv.reshape(d["n_layer"], ctx, kvd)[:, :n_ctx] = v.reshape(d["n_layer"], n_ctx, kvd)
    del k, v
    tok, pos, n = first_tok, n_ctx, 0
    t = time.perf_counter()
    while (n < 2 or time.perf_counter() - t < budget_s) and n < 60:
        m.forward(tok, pos, True)
        tok = O.argmax(m.logits())
        pos += 1
        n += 1
    dt = time.perf_counter() - t
    m.close()
    return dict(decode_tok_s=round(n / dt, 3), threads=threads, kind="port",
                sample=f"{n} greedy decode forwards at positions {n_ctx}..{n_ctx + n - 1} on the GPU-prefilled KV")


def time_kernel(aotk, kind, rows, cols, iters=200, min_bytes=1 << 30):
    """Mean ms per launch of the matvec over rotated synthetic copies."""
    import numpy as np
    from aotk import abi
    rb = rows * abi.row_bytes(kind, cols)
    copies = max(2, min(64, -(-min_bytes // rb)))
    rng = np.random.default_rng(1)
    # 512 distinct rows of seeded N(0, 0.02) values encoded on the device,
    # repeated to the full row count (the bytes streamed per launch are the
    # full matrix's), uploaded as rotated copies
    base = aotk.quantize_rows(kind, (rng.standard_normal((min(rows, 512), cols)) * 0.02).astype(np.float32))
    raw = np.resize(base, (rows, base.shape[1]))
    ws = [aotk.Weight(kind, raw, rows, cols) for _ in range(copies)]
    del raw
    xv = rng.standard_normal(cols).astype(np.float32)
    aotk.time_matvec(ws, xv, copies)  # warm-up
    ms = aotk.time_matvec(ws, xv, max(iters, copies))
    for w in ws:
        w.free()
    return ms, copies


def extra_config(aotk, configs, name, n_ctx, steps, chunk=64, cpu_s=0.0):
    """Another benchmark config as written: the KV cache prefilled by a
    random-id prompt of n_ctx tokens through the batched prompt path
    (app.rs:474-485, chunks of 64; timed: prefill tok/s), then `steps`
    greedy decode forwards (timed: decode tok/s). HBM fractions count the
    weights plus the attended KV rows per token against the 8 TB/s peak; the
    prefill's counts every chunk's pass over the layer weights."""
    spec = configs.build(name)
    model = aotk.Model(spec, seed=SEED)
    st = aotk.State(model, n_ctx + steps + 2, chunk)
    toks = configs.prompt_tokens(2, n_ctx, spec.d["vocab"])
    aotk.sync()
    t = time.perf_counter()
    st.prompt(toks, batch=chunk)
    aotk.sync()
    t_pre = time.perf_counter() - t
    # warm-up and graph capture past the timed positions, then the prompt's
    # last forward again (the same KV row, the prompt-end logits back), so
    # that the timed stream is the config's own from its first token
    st.generate(n_ctx + steps, 2)
    st.forward(toks[-1], n_ctx - 1, True)
    aotk.sync()
    t = time.perf_counter()
    gen = st.generate(n_ctx, steps + 1)
    aotk.sync()
    dt = time.perf_counter() - t
    wb = model.weight_bytes()
    kvb = kv_bytes_per_token(spec, n_ctx, steps)
    tok_s = steps / dt
    pre_b = -(-n_ctx // chunk) * layer_weight_bytes(spec) + spec.out_tensor.len
    res = dict(decode_tok_s=round(tok_s, 2), prefill_tok_s=round(n_ctx / t_pre, 1), prefill_s=round(t_pre, 3),
               context=n_ctx, steps=steps, weight_GB=round(wb / 1e9, 3), kv_GB_per_token=round(kvb / 1e9, 4),
               decode_hbm_GBs=round((wb + kvb) * tok_s / 1e9, 1),
               decode_hbm_frac=round((wb + kvb) * tok_s / 1e9 / HBM_PEAK_GBS, 4),
               prefill_hbm_frac=round(pre_b / t_pre / 1e9 / HBM_PEAK_GBS, 4), greedy_head=gen[:8],
               note=f"{n_ctx}-token random-id prompt in {chunk}-token chunks, then {steps} greedy decode tokens")
    if cpu_s > 0:
        blob = model.download()
        res["cpu_baseline"] = cpu_decode_from_gpu_kv(spec, blob, st, n_ctx, gen[0], cpu_s)
        del blob
    st.free()
    model.free()
    return res


def tinyllama_config(aotk, configs, reps=20):
    """configs[0] as written: TinyLlama-1.1B shape Q4_K_M, a 6-token
    random-id prompt (batch 1 forward_batch), then 32 greedy tokens (31
    forwards). The config is milliseconds long, so it runs `reps` times
    (same positions, the KV rows rewritten) and the median is reported."""
    import statistics
    name = "tinyllama-1.1b-q4km"
    spec = configs.build(name)
    model = aotk.Model(spec, seed=SEED)
    st = aotk.State(model, 6 + 32, 64)
    toks = configs.prompt_tokens(1, 6, spec.d["vocab"])
    st.prompt(toks, batch=64)
    st.generate(6, 32)  # warm-up and graph capture
    tp, tg = [], []
    for _ in range(reps):
        aotk.sync()
        t = time.perf_counter()
        st.prompt(toks, batch=64)
        aotk.sync()
        tp.append(time.perf_counter() - t)
        t = time.perf_counter()
        gen = st.generate(6, 32)
        aotk.sync()
        tg.append(time.perf_counter() - t)
    wb = model.weight_bytes()
    kvb = kv_bytes_per_token(spec, 6, 31)
    tok_s = 31 / statistics.median(tg)
    st.free()
    model.free()
    return dict(prompt_tok_s=round(6 / statistics.median(tp), 1), decode_tok_s=round(tok_s, 1),
                weight_GB=round(wb / 1e9, 4), decode_hbm_GBs=round((wb + kvb) * tok_s / 1e9, 1),
                decode_hbm_frac=round((wb + kvb) * tok_s / 1e9 / HBM_PEAK_GBS, 4), greedy_head=gen[:8],
                note=f"6-token random-id prompt, then 32 greedy tokens (31 forwards); median of {reps} runs")


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC
    summary (FETCH_SIZE / WRITE_SIZE scaled by a copy kernel of known size),
    or None when no summary for that kernel exists."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    return t.get("traffic_bytes") if t.get("kernel") == kernel else None


def cpu_baseline(spec, blob, n_prompt, chunk, budget_s):
    """The oracle (the restated avx2+f16c kernels) on this host's cores, on
    the same workload as the GPU line: the same n_prompt-token prompt in
    chunks of `chunk` (timed: prompt tok/s), then greedy decode from
    position n_prompt until the time budget is spent, with the reference's
    default thread count min(cores, 8) (app.rs:214-216); then the same decode
    for half the budget on all cores. tok/s as the reference's stats line."""
    from oracle import oracle as O
    from aotk import configs
    cores = os.cpu_count() or 1

    def decode(m, threads, budget):
        tok = O.argmax(m.logits())
        pos, n = n_prompt, 0
        t = time.perf_counter()
        while time.perf_counter() - t < budget and n < 400:
            m.forward(tok, pos, True)
            tok = O.argmax(m.logits())
            pos += 1
            n += 1
        return n, time.perf_counter() - t

    threads = min(cores, 8)
    ctx = n_prompt + 420
    toks = configs.prompt_tokens(1, n_prompt, spec.d["vocab"])
    m = O.Model(spec, blob, ctx, max_batch=chunk, n_threads=threads, kernels=1)
    t = time.perf_counter()
    m.prompt(toks, batch=chunk)
    tp = time.perf_counter() - t
    n, tg = decode(m, threads, budget_s)
    m.close()
    all_cores = None
    if cores > threads:
        m = O.Model(spec, blob, ctx, max_batch=chunk, n_threads=cores, kernels=1)
        m.prompt(toks, batch=chunk)
        n2, tg2 = decode(m, cores, budget_s / 2)
        m.close()
        all_cores = dict(decode_tok_s=round(n2 / tg2, 3), threads=cores)
    return dict(value=round(n / tg, 3), unit="tok/s", cores=threads, kind="port",
                sample=f"{spec.cfg.get('name', 'llama3-8b-q4km')}: the same {n_prompt}-token prompt in {chunk}-token "
                       f"chunks ({n_prompt / tp:.2f} prompt tok/s), then {n} greedy decode forwards at positions "
                       f"{n_prompt}..{n_prompt + n - 1}, avx2+f16c kernels, {threads} threads",
                host_cpu=cpu_model(), host_cores=cores, prompt_tok_s=round(n_prompt / tp, 3), all_cores=all_cores)


def micro_only():
    """Short program for counter and trace runs: 200 launches of the Q4_K
    14336x4096 matvec over rotated copies, one device-to-device copy of 256
    MiB (the calibration kernel: it reads and writes exactly 256 MiB), then
    the HBM ceiling probes of the bench line."""
    import aotk
    from aotk import abi
    ms, copies = time_kernel(aotk, abi.Q4_K, 14336, 4096)
    n = 256 << 20
    src, dst = aotk.DeviceBuffer(n), aotk.DeviceBuffer(n)
    aotk.copy_dev(dst, src, n)
    aotk.sync()
    src.free()
    dst.free()
    log(f"q4_K 14336x4096: {ms * 1e3:.2f} us over {copies} copies; copied {n} bytes")
    log(f"hbm ceiling: {hbm_ceiling(aotk)}")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", default="llama3-8b-q4km")
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--chunk", type=int, default=64)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--extra-steps", type=int, default=256, help="decode tokens of the Qwen3 / Gemma-3 lines")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-extra-seconds", type=float, default=8.0,
                    help="CPU decode sample per long-context config (0: none)")
    ap.add_argument("--no-micro", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the Qwen3 / Gemma-3 decode lines")
    ap.add_argument("--micro-only", action="store_true",
                    help="only the Q4_K 14336x4096 matvec and a 256 MiB device copy (for rocprofv3 --pmc runs)")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one MI355X; the hot path has no multi-GPU mode "
              "(sharding is a design note only). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import aotk
    from aotk import abi, configs
    aotk.init(0)
    if a.micro_only:
        micro_only()
        return

    spec = configs.build(a.config)
    spec.cfg["name"] = a.config
    t = time.perf_counter()
    model = aotk.Model(spec, seed=SEED)
    log(f"{a.config}: weights synthesised in HBM in {time.perf_counter() - t:.2f} s "
        f"({spec.blob_len / 1e9:.2f} GB blob)")
    ctx = a.prompt + a.warmup + a.steps + 2
    st = aotk.State(model, ctx, max_batch=a.chunk)
    toks = configs.prompt_tokens(1, a.prompt, spec.d["vocab"])

    st.prompt(toks, batch=a.chunk)  # untimed first pass (page-in, first launches)
    aotk.sync()
    t = time.perf_counter()
    st.prompt(toks, batch=a.chunk)
    aotk.sync()
    t_prompt = time.perf_counter() - t
    prompt_tok_s = a.prompt / t_prompt
    log(f"prompt: {a.prompt} tokens in {t_prompt * 1e3:.1f} ms ({prompt_tok_s:.1f} tok/s)")

    warm = st.generate(a.prompt, a.warmup + 1)
    aotk.sync()
    t = time.perf_counter()
    gen = st.generate(a.prompt + a.warmup, a.steps + 1)
    aotk.sync()
    t_gen = time.perf_counter() - t
    tok_s = a.steps / t_gen
    wbytes = model.weight_bytes()
    # int8 MFMA work of the prompt: 2 * tokens * the layer matrices' weights
    # (the logits of a chunk come from its last row alone, a matvec)
    layer_params = sum(getattr(L, n).rows * getattr(L, n).cols for L in spec.layers
                       for n in ("wq", "wk", "wv", "wo", "gate", "up", "down"))
    prompt_tops = 2.0 * layer_params * prompt_tok_s / 1e12
    log(f"decode: {a.steps} forwards in {t_gen * 1e3:.1f} ms ({tok_s:.1f} tok/s, "
        f"{wbytes * tok_s / 1e9:.0f} GB/s of weights)")

    n_chunks = -(-a.prompt // a.chunk)
    prompt_bytes = n_chunks * layer_weight_bytes(spec) + spec.out_tensor.len
    prompt_hbm_frac = prompt_bytes / t_prompt / 1e9 / HBM_PEAK_GBS
    kvb = kv_bytes_per_token(spec, a.prompt + a.warmup, a.steps)
    ceiling = None if a.no_micro else hbm_ceiling(aotk)
    roofline = None
    micro = {}
    kinds_micro = {}
    if not a.no_micro:
        shapes = [(4096, 4096), (14336, 4096), (4096, 14336), (128256, 4096)]

        def measure(kind, rows, cols):
            ms, copies = time_kernel(aotk, kind, rows, cols)
            b = matvec_bytes(kind, rows, cols)
            gbs = b / (ms * 1e-3) / 1e9
            log(f"{abi.KIND_NAMES[kind]} matvec {rows}x{cols}: {ms * 1e3:.2f} us, {gbs:.0f} GB/s")
            return dict(us=round(ms * 1e3, 2), GBs=round(gbs, 1), frac=round(gbs / HBM_PEAK_GBS, 4), copies=copies)

        for rows, cols in shapes:
            micro[f"{rows}x{cols}"] = measure(abi.Q4_K, rows, cols)
        # every other kind at every shape
        for kind in (abi.Q6_K, abi.Q5_K, abi.Q8_0, abi.Q4_0, abi.Q5_0, abi.F16, abi.BF16):
            kinds_micro[abi.KIND_NAMES[kind]] = {f"{r}x{c}": measure(kind, r, c) for r, c in shapes}
        dom = micro["14336x4096"]
        roofline = dict(bound="hbm", achieved=dom["GBs"], peak=HBM_PEAK_GBS, unit="GB/s", frac=dom["frac"],
                        traffic=measured_traffic("k_mv_kq<Q4_K> 14336x4096"),
                        kernel="k_mv_kq<Q4_K> 14336x4096 (ffn gate/up shape)",
                        bytes_per_launch=matvec_bytes(abi.Q4_K, 14336, 4096), us_per_launch=dom["us"],
                        frac_of_read_ceiling=round(dom["GBs"] / ceiling["read_33MB_GBs"], 4))

    extra = {}
    if not a.no_extra:
        extra["tinyllama-1.1b-q4km"] = tinyllama_config(aotk, configs)
        log(f"tinyllama-1.1b-q4km: prompt {extra['tinyllama-1.1b-q4km']['prompt_tok_s']} tok/s, "
            f"decode {extra['tinyllama-1.1b-q4km']['decode_tok_s']} tok/s")
        for name, n_ctx in (("qwen3-8b-q8_0", 4096), ("gemma3-4b-q5km", 8192)):
            extra[name] = extra_config(aotk, configs, name, n_ctx, a.extra_steps,
                                       cpu_s=0.0 if a.no_cpu else a.cpu_extra_seconds)
            log(f"{name}: prefill {n_ctx} tokens {extra[name]['prefill_tok_s']} tok/s, "
                f"{extra[name]['decode_tok_s']} tok/s decode at {n_ctx}+ context")

    cpu = None
    if not a.no_cpu:
        log("cpu baseline: downloading the weights and running the oracle ...")
        blob = model.download()
        st.free()
        cpu = cpu_baseline(spec, blob, a.prompt, a.chunk, a.cpu_seconds)
        log(f"cpu baseline: {cpu['value']} tok/s on {cpu['cores']} threads ({cpu['host_cpu']})")
        if not a.no_micro:
            cpu["matvec"] = cpu_matvec_cells(aotk, [(4096, 4096), (14336, 4096), (4096, 14336), (128256, 4096)],
                                             (abi.Q4_K, abi.Q6_K, abi.Q5_K, abi.Q8_0, abi.Q4_0, abi.Q5_0, abi.F16,
                                              abi.BF16))
            log(f"cpu matvec GB/s: {cpu['matvec']['GBs']}")
        cpu["other_configs"] = {k: v.get("cpu_baseline") for k, v in extra.items() if v.get("cpu_baseline")}

    line = {
        "metric": "decode tok/s + Q4_K matvec HBM GB/s (frac of peak); prompt tok/s, 1 MI355X",
        "value": round(tok_s, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(t_gen / a.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": f"{a.config}: {a.prompt}-token random-id prompt in {a.chunk}-token chunks, "
                               f"then greedy decode (batch 1)",
                   "prompt_tokens": a.prompt, "chunk": a.chunk, "seed": SEED},
        "prompt_tok_s": round(prompt_tok_s, 2),
        "prompt_int8_TOPs": round(prompt_tops, 1),
        "prompt_int8_frac": round(prompt_tops / INT8_PEAK_TOPS, 4),
        "prompt_hbm_frac": round(prompt_hbm_frac, 4),
        "prompt_hbm_bytes": prompt_bytes,
        "decode_kv_bytes_per_token": round(kvb),
        "decode_hbm_frac": round((wbytes + kvb) * tok_s / 1e9 / HBM_PEAK_GBS, 4),
        "hbm_ceiling": ceiling,
        "decode_weight_bytes_per_token": wbytes,
        "decode_weight_GBs": round(wbytes * tok_s / 1e9, 1),
        "q4k_matvec": micro,
        "matvec_kinds": kinds_micro,
        "other_configs": extra,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "greedy_head": gen[:8],
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
