"""bench.py's contract on the CPU: one GPU only (--gpus above 1 exits with a
message, before touching a GPU), and the committed counter summaries it
reads for the roofline's `traffic` parse with the keys it needs."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


@pytest.mark.parametrize("n", [2, 8])
def test_more_than_one_gpu_refused(n):
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", str(n)], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2, r
    assert "one GPU only" in r.stderr and r.stdout == ""


@pytest.mark.parametrize("kernel,name", sorted(bench.TRAFFIC_PROFILES.items()))
def test_traffic_profiles_parse(kernel, name):
    path = os.path.join(ROOT, "profiles", name)
    assert os.path.exists(path), path
    vals = {}
    with open(path) as f:
        for line in f:
            if ":" in line and not line.startswith("#"):
                k, v = line.split(":", 1)
                vals[k.strip()] = v.strip()
    assert vals["kernel"] == kernel
    assert vals["workload"] == "19x19 10x128 batch 256"
    assert float(vals["hbm_bytes_per_launch"]) > 0
    assert float(vals["fetch_scale"]) > 0 and float(vals["write_scale"]) > 0
    # traffic_from_profile gives the figure back for the summary's own keys,
    # and nothing for another build's convolution or another workload.
    got = bench.traffic_from_profile(vals["workload"], vals["kernels"], kernel)
    assert got == float(vals["hbm_bytes_per_launch"])
    assert bench.traffic_from_profile(vals["workload"], "00000000", kernel) is None
    assert bench.traffic_from_profile("9x9 6x64 batch 64", vals["kernels"], kernel) is None
