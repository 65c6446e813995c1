"""Build libaotk.so for gfx950 in-tree with hipcc (no CMake, no JIT cache).

    python aot-llm_amd/build.py [--jobs N]

Compiles every csrc/*.hip to an object in parallel and links the shared
library next to this file, where aotk/abi.py loads it.
"""
import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "libaotk.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950",
    # bit-exactness: no implicit FMA contraction, IEEE division and sqrt
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    # never emit packed-FP32 VALU ops (they are avoided on this pool)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # matrix-core results in VGPRs (the f32 folds read them directly; the
    # AGPR form costs one v_accvgpr_read per value)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unused-result",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def compile_one(src):
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC] + FLAGS + ["-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    return src, obj, r.returncode, r.stdout + r.stderr


def build(jobs=8, verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    objs = []
    errors = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        for src, obj, rc, log in ex.map(compile_one, sources()):
            msgs = [ln for ln in log.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
            if rc != 0:
                errors.append(f"--- {src}\n" + "\n".join(msgs))
            elif verbose and msgs:
                print("\n".join(msgs))
            objs.append(obj)
    if errors:
        raise RuntimeError("hipcc failed:\n" + "\n".join(errors))
    tmp = OUT + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 4))
    ap.add_argument("-v", "--verbose", action="store_true")
    a = ap.parse_args()
    try:
        print(build(a.jobs, a.verbose))
    except RuntimeError as e:
        print(e, file=sys.stderr)
        sys.exit(1)
