"""The `hip` name sites (oracle/hip_names.patch) against the reference's own
sources, on the CPU: every hunk applies to a scratch copy (src/build_info.cpp
included, which needs a CMake-generated include and so is never compiled
here), each site the patch names carries its hip line, and every patched
source passes the compiler's syntax check with AZ_USE_HIP (the coordinator's
memory check through checkHipInferenceMemory among them). Skipped where the
reference tree is absent (it is on the build host only)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = os.environ.get("AZGO_REFERENCE", "/root/reference")
PATCH = os.path.join(ROOT, "oracle", "hip_names.patch")
SOURCES = ["inference_hub", "backend", "arena", "config", "engines", "coordinator", "build_info"]
HEADERS = ["engines", "build_info"]

pytestmark = pytest.mark.skipif(not os.path.exists(os.path.join(REF, "src", "engines.cpp")),
                                reason="the reference tree is not present")


@pytest.fixture(scope="module")
def patched(tmp_path_factory):
    d = tmp_path_factory.mktemp("patched")
    os.makedirs(d / "src")
    os.makedirs(d / "include" / "azgo")
    for s in SOURCES:
        shutil.copy(os.path.join(REF, "src", s + ".cpp"), d / "src")
    for h in HEADERS:
        shutil.copy(os.path.join(REF, "include", "azgo", h + ".hpp"), d / "include" / "azgo")
    shutil.copy(os.path.join(ROOT, "alphazero-go_amd", "host", "hip.hpp"), d / "include" / "azgo" / "hip.hpp")
    with open(PATCH) as f:
        r = subprocess.run(["patch", "-p1", "--forward", "-d", str(d)], stdin=f, capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "offset" not in r.stdout and "fuzz" not in r.stdout, r.stdout   # every hunk where it says
    return d


def _read(d, rel):
    with open(d / rel) as f:
        return f.read()


def test_every_site_names_hip(patched):
    eng = _read(patched, "src/engines.cpp")
    assert 'e.backend != "hip"' in eng and "(expected naive|blas|metal|cuda|hip)" in eng
    assert '"hip_workers"' in eng and "m.hipWorkers" in eng and "machine.hipWorkers" in eng
    assert 'if (backend == "hip") f += "; " + hipDescription();' in eng
    assert "int metalWorkers = 0, cudaWorkers = 0, hipWorkers = 0" in _read(patched, "include/azgo/engines.hpp")
    co = _read(patched, "src/coordinator.cpp")
    assert "checkHipInferenceMemory(cfg_.netConfig(), g)" in co and "#ifdef AZ_USE_HIP" in co
    assert co.count('"hip"') >= 6   # hub counts, memory check, remote workers, three CPU-class sites
    assert 'if (hipBuilt()) return "hip";' in _read(patched, "src/build_info.cpp")
    assert 'backend == "hip"' in _read(patched, "src/inference_hub.cpp")
    assert 'name == "hip"' in _read(patched, "src/backend.cpp")
    assert 'backend == "hip"' in _read(patched, "src/arena.cpp")
    assert 'v == "hip"' in _read(patched, "src/config.cpp")


@pytest.mark.parametrize("source", [s for s in SOURCES if s != "build_info"])
def test_patched_source_compiles(patched, source):
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-DAZ_USE_HIP", "-I", str(patched / "include"),
                        "-I", os.path.join(REF, "include"), str(patched / "src" / (source + ".cpp"))],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
