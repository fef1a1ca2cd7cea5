"""Test setup: the `gpu` marker, import paths for the oracle (what results are checked against)
and the backend's Python binding, and shared fixtures."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("oracle", "alphazero-go_amd"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X); runs the HIP library's kernels")
    _ensure_built()


def _ensure_built():
    """Builds what the tests load when a fresh checkout lacks it: the oracle
    (gcc, seconds), the workload generator (g++) and, where hipcc exists, the
    HIP library. A machine without the toolchain needs them prebuilt."""
    import subprocess
    if not os.path.exists(os.path.join(ROOT, "oracle", "liboracle.so")):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "oracle"], check=True)
    pkg = os.path.join(ROOT, "alphazero-go_amd")
    need_workload = not os.path.exists(os.path.join(pkg, "libazgo_workload.so"))
    need_hip = not os.path.exists(os.path.join(pkg, "libazgo_hip.so")) and os.path.exists("/opt/rocm/bin/hipcc")
    if need_workload or need_hip:
        import build as pkg_build
        if need_workload:
            pkg_build.build_workload()
        if need_hip:
            pkg_build.build()


@pytest.fixture(scope="session")
def hip():
    """The backend's binding, with the GPU checked once: a GPU test fails
    (not skips) when the native library or the device is unusable."""
    import azgo_hip
    ok, why = azgo_hip.available()
    if not ok:
        pytest.fail(f"no usable gfx950 GPU: {why}")
    return azgo_hip
