"""The inference pass on generation-0 networks as the reference's trainer
makes them: Network(cfg, 1)'s weights with the batch-norm running
statistics of calibrateBatchNorm (src/bn_calibration.cpp:33-45, the
trainer's seed, src/trainer.cpp:559; tests/golden/calibrated_bn.npz). These
are normalised networks (|logit| of a few units, values inside (-1, 1)), so
the parity bar applies as written, at every benchmark shape including
the 19x19 headline: max-abs 1e-4 on logits and on values against the blas
restatement of Network::infer, and argmax agreement over legal moves of at
least 99.9%.

Also end to end from a file: checkpoints the reference's saveNetwork wrote
(tests/golden/gen0_*.azn), loaded by azh_create_from_checkpoint, against the
reference's own Network::infer of the same files (gen0_infer.npz).
"""
import os

import numpy as np
import pytest

import oracle as O
from _util import GOLDEN, calibrated_network, parity_report, to_hip_cfg, bitwise_equal

pytestmark = pytest.mark.gpu

TOL = 1e-4   # max-abs on logits and values (the parity bar)

# (calibration tag, network config, GPU batch, positions checked on the CPU).
# Every position of every batch is checked; the 20x256 net's 512 on a pool
# of threads (each position's outputs depend on its own input only).
CASES = [
    ("1", O.WORKLOADS[1].cfg, 8, 8),
    ("2", O.WORKLOADS[2].cfg, 64, 64),
    ("3", O.WORKLOADS[3].cfg, 256, 256),
    ("3", O.WORKLOADS[3].cfg, 1, 1),
    ("3", O.WORKLOADS[3].cfg, 8, 8),
    ("3", O.WORKLOADS[3].cfg, 32, 32),
    ("3v256", O.make_cfg(19, 10, 128, value_hidden=256), 64, 64),
    ("5", O.WORKLOADS[5].cfg, 512, 512),
]


def _workload_for(cfg):
    for w in O.WORKLOADS.values():
        if (w.cfg.board, w.cfg.blocks, w.cfg.filters) == (cfg.board, cfg.blocks, cfg.filters):
            return w
    raise KeyError(cfg)


@pytest.mark.parametrize("tag,cfg,B,check", CASES,
                         ids=[f"{c[0]}-b{c[2]}" for c in CASES])
def test_calibrated_parity(hip, tag, cfg, B, check):
    net = calibrated_network(tag, cfg)
    w = _workload_for(cfg)
    inp, legal = O.workload_inputs(w, B)
    with hip.Runner(to_hip_cfg(hip, cfg), net.tensors(), B, 1) as r:
        logits, values = r.infer(inp)
    assert np.isfinite(logits).all() and np.isfinite(values).all()
    idx = np.linspace(0, B - 1, check).round().astype(int)
    blas = O.threaded(lambda x: O.forward(net, x, O.BLAS), inp[idx], 8)
    rep = parity_report(logits[idx], values[idx], blas[0], blas[1], legal[idx])
    rep["max_abs_logit"] = float(np.abs(blas[0]).max())
    # Context: the reference's two CPU backends differ by about as much.
    few = idx[:min(4, check)]
    naive = O.forward(net, inp[few], O.NAIVE)
    rep["cpu_naive_vs_blas_logits"] = float(np.abs(naive[0].astype(np.float64) - blas[0][:len(few)]).max())
    print(f"calibrated {tag} B={B} (checked {check}): {rep}")
    assert rep["logits_maxabs"] <= TOL, rep
    assert rep["values_maxabs"] <= TOL, rep
    assert rep["argmax_agree"] >= 0.999, rep


def test_calibrated_vs_double_within_cpu_gap(hip):
    """The reference's bar for its CUDA port (tests/test_cuda.cpp:804-849) on
    the calibrated headline network: the GPU's gap to the double-precision
    pass within max(1e-5, 2x the CPU backends' own gap), never above 5e-5."""
    net = calibrated_network("3")
    inp, _ = O.workload_inputs(O.WORKLOADS[3], 4)
    with hip.Runner(to_hip_cfg(hip, net.cfg), net.tensors(), 4, 1) as r:
        got = r.infer(inp)
    dbl = O.forward_double(net, inp)
    cpu = max(O.max_err(O.forward(net, inp, m)[0], dbl[0]) for m in (O.BLAS, O.NAIVE))
    gpu = O.max_err(got[0], dbl[0])
    print(f"maxErr vs double: gpu {gpu:.3g}, cpu backends {cpu:.3g}")
    assert gpu <= min(5e-5, max(1e-5, 2 * cpu))
    assert float(np.abs(got[1].astype(np.float64) - dbl[1]).max()) <= 1e-5


@pytest.mark.parametrize("tag,own", [("4x32", False), ("2x16_own", True)])
def test_checkpoint_end_to_end(hip, tag, own):
    path = os.path.join(GOLDEN, f"gen0_5x5_{tag}.azn")
    g = np.load(os.path.join(GOLDEN, "gen0_infer.npz"))
    inp = g["input"]
    B = inp.shape[0]
    with hip.Runner.from_checkpoint(path, B, 1) as r:
        assert bool(r.cfg.ownership) == own
        got = r.infer(inp, ownership=own)
    rep = parity_report(got[0], got[1], g[f"{tag}/logits"], g[f"{tag}/values"], g["legal"])
    print(f"checkpoint {tag}: {rep}")
    assert rep["logits_maxabs"] <= TOL and rep["values_maxabs"] <= TOL and rep["argmax_agree"] >= 0.999, rep
    if own:
        d = float(np.abs(got[2].astype(np.float64) - g[f"{tag}/ownership"]).max())
        assert d <= TOL, d
    # The same weights through azh_create give the same bits.
    cfg, tensors = hip.checkpoint_read(path)
    with hip.Runner(cfg, tensors, B, 1) as r:
        again = r.infer(inp, ownership=own)
    for a, b in zip(got, again):
        assert bitwise_equal(a, b)
