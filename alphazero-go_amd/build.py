"""Builds libazgo_hip.so in place (gfx950 only) with hipcc.

Every source is compiled with -ffp-contract=off (no multiply-add the source
does not spell out: the BN epilogue and the host-side BN fold round each
operation separately) and with packed FP32 instructions disabled.
"""
from __future__ import annotations

import hashlib
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libazgo_hip.so")
SOURCES = ["azh_kernels.hip", "azh_runtime.hip"]
HEADERS = ["azh_kernels.hpp", os.path.join("..", "..", "include", "azgo_hip.h")]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         # The conv kernels' step streams (up to 9 taps x 23 column groups
         # per chunk) are unrolled whole; the default size limit for a
         # pragma-requested unroll stops short of that.
         "-mllvm", "-pragma-unroll-threshold=100000",
         "-I", os.path.join(ROOT, "include"), "-Wall"]


def kernel_hash():
    """A hash of the kernel sources, headers and flags: two builds whose
    hashes match run the same GPU arithmetic."""
    h = hashlib.sha256()
    for f in SOURCES + HEADERS:
        with open(os.path.join(CSRC, f), "rb") as fh:
            h.update(fh.read())
    h.update(" ".join(FLAGS).encode())
    return h.hexdigest()[:8]


def build(verbose=False):
    build_dir = os.path.join(HERE, "_build")
    os.makedirs(build_dir, exist_ok=True)
    defs = [f'-DAZH_KERNEL_HASH="{kernel_hash()}"']

    def compile_one(src):
        obj = os.path.join(build_dir, src.replace(".hip", ".o"))
        cmd = [HIPCC] + FLAGS + defs + ["-c", os.path.join(CSRC, src), "-o", obj]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
        if verbose and r.stderr.strip():
            print(r.stderr, file=sys.stderr)
        return obj

    with ThreadPoolExecutor(len(SOURCES)) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs + ["-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


def build_workload():
    """libazgo_workload.so: the seeded benchmark workloads (host C++)."""
    src = os.path.join(HERE, "workload", "azgo_workload.cpp")
    out = os.path.join(HERE, "libazgo_workload.so")
    cmd = [os.environ.get("CXX", "g++"), "-std=c++17", "-O2", "-ffp-contract=off", "-fPIC", "-shared",
           src, "-o", out + ".tmp"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"workload build failed:\n{r.stderr}")
    os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
    print(build_workload())
