"""Whole-batch launches of the stem and the heads on one stream, for
rocprofv3 --kernel-trace: in a pass of a large batch they run as two
concurrent half-batch launches, whose traced durations overlap the other
half's work. Random weights (BN variances in [0.5, 1.5]) and a random
trunk; the network shape and batch are arguments.

    python3 alphazero-go_amd/profile_stem_heads.py [--board 19] [--blocks 10]
        [--filters 128] [--value-hidden 64] [--batch 256] [--iters 10]
"""
import argparse
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import azgo_hip  # noqa: E402

ap = argparse.ArgumentParser()
ap.add_argument("--board", type=int, default=19)
ap.add_argument("--history", type=int, default=8)
ap.add_argument("--blocks", type=int, default=10)
ap.add_argument("--filters", type=int, default=128)
ap.add_argument("--value-hidden", type=int, default=64)
ap.add_argument("--batch", type=int, default=256)
ap.add_argument("--iters", type=int, default=10)
a = ap.parse_args()

cfg = azgo_hip.net_cfg(a.board, a.history, a.blocks, a.filters, a.value_hidden)
rng = np.random.default_rng(1)
tensors = {}
for name, floats in azgo_hip.tensor_spec(cfg):
    lo, hi = (0.5, 1.5) if name.endswith("runVar") else (-0.05, 0.05)
    tensors[name] = rng.uniform(lo, hi, floats).astype(np.float32)
A = a.board * a.board
planes = cfg.planes
with azgo_hip.Runner(cfg, tensors, a.batch, 1) as r:
    trunk = rng.uniform(0, 2, (a.batch, a.filters, A)).astype(np.float32)
    for _ in range(a.iters):
        r.probe_heads(trunk)
ms = azgo_hip.time_conv3x3(a.batch, a.board, planes, a.filters, -1, a.iters)
print(f"{a.board}x{a.board} {a.blocks}x{a.filters} batch {a.batch}: heads x {a.iters} on a given trunk; "
      f"stem ({planes} planes -> {a.filters}) {ms * 1e3:.1f} us per launch", flush=True)
