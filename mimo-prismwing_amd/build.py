"""Builds the gfx950 library libpwfp8.so in-tree with hipcc (no CMake, no JIT cache).

Usage: python mimo-prismwing_amd/build.py [--jobs N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "prismwing_amd")
LIB = os.path.join(OUT_DIR, "libpwfp8.so")
OBJ_DIR = os.path.join(HERE, "_build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["pw_linear.hip", "pw_bf16.hip", "pw_moe.hip", "pw_moe_a.hip", "pw_moe_b.hip", "pw_prefill.hip", "pw_router.hip",
           "pw_synth.hip", "pw_checkpoint.cpp",
           "pw_runtime.cpp"]

FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    # no packed FP32 instructions anywhere (some of their forms misbehave on these parts)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # IEEE division (the reference's quantiser and sigmoid divide correctly rounded)
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # a*b+c is never contracted implicitly; fused multiply-adds are written out where wanted
    "-ffp-contract=off",
    "-Wall", "-Wno-unused-function",
]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{proc.stderr}")
    return obj


def build(jobs: int = 6, verbose: bool = True) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    sources = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=6)
    args = ap.parse_args()
    try:
        build(args.jobs)
    except RuntimeError as exc:
        print(exc, file=sys.stderr)
        sys.exit(1)
