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
SOURCES = ["azh_kernels.hip", "azh_positions.hip", "azh_runtime.hip", "azh_small_tower.hip"]
# The 3x3 convolution is one template instantiated per (board size,
# workgroup shape): azh_conv_inst.hip is compiled once per pair, so the
# fully unrolled kernels build in parallel.
CONV_INST = "azh_conv_inst.hip"
CONV_HEADERS = ["azh_conv.hpp", "azh_conv_iface.hpp", "azh_stem.hpp"]
BOARD_SIZES = (5, 9, 13, 19)   # conv3x3Supported
RESIDENT_BOARD_SIZES = (19,)   # residentTowerSupported
HEADERS = CONV_HEADERS + ["azh_kernels.hpp", "azh_heads.hpp", os.path.join("..", "..", "include", "azgo_hip.h")]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         # The conv kernels' step streams (up to 9 taps x 23 column groups
         # per chunk) are unrolled whole; the default size limit for a
         # pragma-requested unroll stops short of that.
         "-mllvm", "-pragma-unroll-threshold=100000",
         "-I", os.path.join(ROOT, "include"), "-Wall"]


def _hash(files):
    h = hashlib.sha256()
    for f in files:
        with open(os.path.join(CSRC, f), "rb") as fh:
            h.update(fh.read())
    # The include directory by its place in the tree, not its absolute path:
    # the header's text is hashed with the sources, so two checkouts of the
    # same files hash alike wherever they are.
    h.update(" ".join(FLAGS).replace(ROOT, "<repo>").encode())
    return h.hexdigest()[:8]


def kernel_hash():
    """A hash of every kernel source, header and flag: two builds whose
    hashes match run the same GPU arithmetic."""
    return _hash(SOURCES + [CONV_INST] + HEADERS)


def conv_hash():
    """The same over the 3x3 convolution's sources only: a profile of the
    convolution stays valid while this matches."""
    return _hash([CONV_INST] + CONV_HEADERS)


def conv_tiling_count():
    """Entries of kConvTilings (azh_conv_iface.hpp)."""
    text = open(os.path.join(CSRC, "azh_conv_iface.hpp")).read()
    body = text[text.index("kConvTilings[] = {") + len("kConvTilings[] = {"):]
    body = body[:body.index("};")]
    return body.count("{")


def build(verbose=False, jobs=None, incremental=False):
    """Compiles every unit and links libazgo_hip.so. incremental: skip units
    whose object is newer than every source and header (a development aid;
    the default rebuilds everything)."""
    build_dir = os.path.join(HERE, "_build")
    os.makedirs(build_dir, exist_ok=True)
    defs = [f'-DAZH_KERNEL_HASH="{kernel_hash()}"', f'-DAZH_CONV_HASH="{conv_hash()}"']
    units = [(src, src.replace(".hip", ".o"), []) for src in SOURCES]
    for n in BOARD_SIZES:
        for t in range(conv_tiling_count()):
            units.append((CONV_INST, f"azh_conv_{n}_{t}.o", [f"-DAZH_CONV_N={n}", f"-DAZH_CONV_TILING={t}"]))
    for n in RESIDENT_BOARD_SIZES:
        units.append((CONV_INST, f"azh_resident_{n}.o", [f"-DAZH_CONV_N={n}", "-DAZH_RESIDENT_TOWER"]))

    deps = [os.path.join(CSRC, f) for f in SOURCES + [CONV_INST] + HEADERS] + [os.path.abspath(__file__)]
    newest = max(os.path.getmtime(f) for f in deps)

    def compile_one(unit):
        src, obj_name, extra = unit
        obj = os.path.join(build_dir, obj_name)
        if incremental and os.path.exists(obj):
            mine = [os.path.join(CSRC, src)] + [os.path.join(CSRC, h) for h in HEADERS]
            if src == CONV_INST:
                mine = [os.path.join(CSRC, f) for f in [CONV_INST] + CONV_HEADERS] + [os.path.abspath(__file__)]
            else:
                mine += [os.path.abspath(__file__)]
            if os.path.getmtime(obj) > max(os.path.getmtime(f) for f in mine):
                return obj
        cmd = [HIPCC] + FLAGS + defs + extra + ["-c", os.path.join(CSRC, src), "-o", obj]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src} {' '.join(extra)}:\n{r.stderr}")
        if verbose and r.stderr.strip():
            print(r.stderr, file=sys.stderr)
        return obj

    jobs = jobs or max(1, min(16, os.cpu_count() or 1))
    # Biggest units first (19x19 instances), so the pool ends evenly.
    units.sort(key=lambda u: 0 if "N=19" in " ".join(u[2]) else 1)
    with ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(compile_one, units))
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
    print(build(verbose=True, incremental="--incremental" in sys.argv))
    print(build_workload())
