"""Build libkadllm_hip.so for gfx950 with hipcc (in-tree, no JIT cache).

    python -m kadllm_amd.csrc.build [-j N] [--verbose]

Objects go to kadllm_amd/csrc/_build/; the library to kadllm_amd/.
Every build recompiles all sources (a few seconds each, in parallel).
"""

import argparse
import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
LIB_NAME = "libkadllm_hip.so"
ARCH = "gfx950"

CXXFLAGS = [
    "-std=c++17", "-O3", "-fPIC", f"--offload-arch={ARCH}",
    # keep hipcc from forming packed-fp32 instructions (v_pk_*_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
    "-Wno-unused-command-line-argument",
]


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build")
    return path


def _compile(src, obj, verbose):
    cmd = [hipcc(), *CXXFLAGS, "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {os.path.basename(src)}:\n{err}")
    if err.strip() and verbose:
        print(err, flush=True)
    return obj


def build(jobs=None, verbose=False):
    sources = sorted(glob.glob(os.path.join(HERE, "*.hip")))
    if not sources:
        raise RuntimeError("no HIP sources found")
    out_dir = os.path.join(HERE, "_build")
    os.makedirs(out_dir, exist_ok=True)
    objs = [os.path.join(out_dir, os.path.basename(s)[:-4] + ".o") for s in sources]
    jobs = jobs or min(8, os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, s, o, verbose) for s, o in zip(sources, objs)]
        for f in futs:
            f.result()
    lib = os.path.join(PKG, LIB_NAME)
    tmp = lib + ".tmp"
    cmd = [hipcc(), "-shared", f"--offload-arch={ARCH}", "-o", tmp, *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, lib)
    return lib


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    a = ap.parse_args(argv)
    print(build(a.j, a.verbose))


if __name__ == "__main__":
    sys.exit(main())
