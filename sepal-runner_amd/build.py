"""Builds the HIP library of the W8g128 MLP path for gfx950: sepal_mlp/libsepal_mlp_hip.so (in-tree).

Every source is compiled by hipcc for --offload-arch=gfx950 only, with packed FP32 instructions disabled
(-target-feature -packed-fp32-ops) and no fast-math, then linked into one shared library that exports the C ABI of
include/sepal_mlp_hip.h. Objects are compiled in parallel; the library is always rebuilt (the build check runs it on
every call).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "sepal_mlp")
LIB = os.path.join(OUT_DIR, "libsepal_mlp_hip.so")
OBJ_DIR = os.path.join(HERE, "_build")

SOURCES = ["quant.hip", "gemm_w8g.hip", "gemm_q8.hip", "stream.hip", "stack_small.hip", "packed_file.hip", "edge.hip", "capi.cpp"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++20", "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=off", "-Wall", "-Wno-unused-function", "-Wno-unused-variable", "-Wno-unknown-pragmas",
    "-I" + os.path.join(ROOT, "include"), "-I" + SRC,
]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC, *FLAGS, "-x", "hip", "-c", os.path.join(SRC, src), "-o", obj]
    out = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature for this target (ignoring feature)"
    text = "\n".join(l for l in (out.stdout + out.stderr).splitlines() if noise not in l)
    if out.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{text}")
    if text.strip():
        print(text, file=sys.stderr)
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    os.makedirs(OUT_DIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), int(os.environ.get("MAX_JOBS", "8")))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    out = subprocess.run(cmd, capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError("link failed:\n" + out.stdout + out.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
