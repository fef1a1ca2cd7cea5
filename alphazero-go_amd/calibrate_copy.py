"""A plain device-to-device copy of known size, for scaling HBM traffic
counters: run it under rocprofv3 --pmc FETCH_SIZE (or WRITE_SIZE) and
divide the counter's reading by the bytes copied.

    python3 alphazero-go_amd/calibrate_copy.py [--mib 256] [--iters 5]
"""
import argparse
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import azgo_hip  # noqa: E402

ap = argparse.ArgumentParser()
ap.add_argument("--mib", type=int, default=256)
ap.add_argument("--iters", type=int, default=5)
a = ap.parse_args()
nbytes = a.mib << 20
ms = azgo_hip.probe_copy(nbytes, a.iters)
print(f"copied {nbytes} bytes x {a.iters}: {ms / a.iters:.4f} ms each, "
      f"{2 * nbytes / (ms / a.iters * 1e-3) / 1e9:.1f} GB/s read+write", flush=True)
