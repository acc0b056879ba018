"""Builds libhephfp8.so (gfx950 only) in-tree with hipcc.

Each csrc/*.hip file is compiled to an object in parallel, then linked into
hephaestus_amd/libhephfp8.so; bench_csrc/hbm_read.hip (bench.py's plain-read
and MFMA-loop measurement kernels) and bench_csrc/synth.cpp (its seeded
synthetic inputs, host code) become hephaestus_amd/libhephbench.so. Every HIP
compile carries `-Xclang -target-feature -Xclang -packed-fp32-ops`, which keeps
the compiler from forming packed fp32 VALU instructions.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libhephfp8.so")
# measurement kernels and synthetic inputs for bench.py; not the product
BENCH_SRC = os.path.join(PKG, "bench_csrc", "hbm_read.hip")
BENCH_SYNTH = os.path.join(PKG, "bench_csrc", "synth.cpp")
BENCH_LIB = os.path.join(PKG, "libhephbench.so")
CXX = os.environ.get("CXX", "g++")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

CFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *CFLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    synth_obj = os.path.join(BUILD, "synth.o")
    r = subprocess.run([CXX, "-O2", "-std=c++17", "-fPIC", "-Wall", "-ffp-contract=off",
                        "-pthread", "-c", BENCH_SYNTH, "-o", synth_obj],
                       capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{CXX} failed on {BENCH_SYNTH}:\n{r.stdout}\n{r.stderr}")
    bench_obj = _compile(BENCH_SRC)
    tmp = BENCH_LIB + ".tmp"
    r = subprocess.run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-pthread", "-o", tmp,
                        bench_obj, synth_obj], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of {BENCH_LIB} failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, BENCH_LIB)
    if verbose:
        print(f"built {LIB} and {BENCH_LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
