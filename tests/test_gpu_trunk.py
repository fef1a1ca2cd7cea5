"""The trunk of the benchmark's own networks on the GPU: the stem and every
residual block (src/network.cpp:241-272), read back through the trunk probe,
against the oracle's blas trunk (the same arithmetic as its forward pass,
pinned bit for bit to the reference build's trunk by
tests/test_oracle.py::test_trunk_equals_reference_build).

With the benchmark's synthetic batch-norm statistics the 19x19 10x128
network's policy 1x1 conv is negative at every point, so its logits are
exactly the zero bias and its values saturate at -1: the pass's outputs
cannot show whether the trunk is right. The trunk can: maxErr (max|x - ref|
/ max|ref|, tests/test_cuda.cpp:150-171) at most 1e-5, the reference's
whole-network ceiling for its CUDA port (tests/test_cuda.cpp:756-776), at
full depth and at the benchmark's own batch sizes, every row of the
headline batch and a spread of 128 of the 20x256 network's 512.
"""
import numpy as np
import pytest

import oracle as O
from _util import to_hip_cfg

pytestmark = pytest.mark.gpu

MAX_ERR = 1e-5

# (workload tag, GPU batch, rows checked on the CPU)
CASES = [(3, 256, 256), (4, 1, 1), (4, 8, 8), (4, 32, 32), (5, 512, 128)]


@pytest.mark.parametrize("tag,B,check", CASES, ids=[f"w{c[0]}-b{c[1]}" for c in CASES])
def test_full_depth_trunk_on_benchmark_network(hip, tag, B, check):
    w = O.WORKLOADS[tag]
    net = O.init_network(w.cfg)
    inp, _ = O.workload_inputs(w, B)
    with hip.Runner(to_hip_cfg(hip, w.cfg), net.tensors(), B, 1) as r:
        got = r.probe_trunk(inp, w.cfg.blocks)
    assert got.shape == (B, w.cfg.filters, w.cfg.area) and np.isfinite(got).all()
    rows = np.linspace(0, B - 1, check).round().astype(int)
    ref = O.threaded(lambda x: O.trunk(net, x, mode=O.BLAS), inp[rows], 8)
    err = O.max_err(got[rows], ref)
    # The trunk is not degenerate: most of it is positive, and it grows with depth.
    live = float((ref > 0).mean())
    print(f"workload {tag} B={B}: trunk maxErr {err:.3g} over {check} rows, max {ref.max():.4g}, "
          f"{100 * live:.1f}% positive")
    assert live > 0.2 and ref.max() > 10
    assert err <= MAX_ERR, err


def test_trunk_depths_on_headline_network(hip):
    """The same at every depth of the 19x19 10x128 network (the stem alone,
    then each block), on 16 positions: the gap does not grow past the bar
    anywhere along the tower."""
    w = O.WORKLOADS[3]
    net = O.init_network(w.cfg)
    inp, _ = O.workload_inputs(w, 16)
    with hip.Runner(to_hip_cfg(hip, w.cfg), net.tensors(), 16, 1) as r:
        for k in range(w.cfg.blocks + 1):
            got = r.probe_trunk(inp, k)
            ref = O.threaded(lambda x: O.trunk(net, x, k, mode=O.BLAS), inp, 4)
            err = O.max_err(got, ref)
            print(f"depth {k}: maxErr {err:.3g}, max {ref.max():.4g}")
            assert err <= MAX_ERR, (k, err)
