"""Builds liborion_hip.so (gfx950 only) in-tree with hipcc.

Usage: python orionserve-rs_amd/build.py [--jobs N]
"""
import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "liborion_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = [
    "attention_decode.hip",
    "decode_plan.cpp",
    "attention_prefill.hip",
    "prefill_plan.cpp",
    "gemm.hip",
    "elementwise.hip",
    "runtime.cpp",
    "checkpoint.cpp",
    "sampling.hip",
]

CFLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    # Packed FP32 VALU ops are kept out of the generated code on purpose.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
]


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC] + CFLAGS + ["-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    p = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in p.stderr.splitlines() if noise not in l)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build(jobs=None):
    os.makedirs(BUILD, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    # link beside the library, then rename over it: a process that still
    # maps the previous build keeps its (unlinked) copy intact
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"link failed:\n{p.stderr}")
    os.replace(tmp, LIB)
    build_abi_check()
    return LIB


ROOT = os.path.dirname(HERE)
ABI_CHECK_SRC = os.path.join(ROOT, "tests", "abi", "abi_check.cpp")
ABI_CHECK = os.path.join(ROOT, "tests", "abi", "abi_check")


def build_abi_check():
    """The C++ program that calls the C-ABI as a foreign caller would
    (tests/abi/abi_check.cpp): host code only, linked against the library."""
    tmp = ABI_CHECK + ".tmp"
    cmd = ["g++", "-std=c++17", "-O1", "-Wall", "-Wextra", ABI_CHECK_SRC, "-o", tmp,
           "-L" + HERE, "-lorion_hip", "-Wl,-rpath,$ORIGIN/../../orionserve-rs_amd"]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"abi_check build failed:\n{p.stderr}")
    os.replace(tmp, ABI_CHECK)


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    a = ap.parse_args()
    print(build(a.jobs))
