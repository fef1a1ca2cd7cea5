"""The whole inference pass on the GPU, through the C ABI, against the oracle
(the reference's Network::infer restated: src/network.cpp:171-183, 228-309).

Parity per workload (the five benchmark configurations, seeded weights and
boards): max-abs on logits and values against the blas restatement (the
parity bar is 1e-4), maxErr, the gap to the double-precision pass next to
the CPU backends' own gap (tests/test_cuda.cpp:804-849), and argmax agreement
over legal moves (>= 99.9%). Full-size batches are checked through
properties: batch independence and repeatability, bit for bit.
"""
import os
import threading
import time

import numpy as np
import pytest

import oracle as O
from _util import bitwise_equal, parity_report, to_hip_cfg

pytestmark = pytest.mark.gpu


def _runner(hip, net, max_batch, slots=1):
    return hip.Runner(to_hip_cfg(hip, net.cfg), net.tensors(), max_batch, slots)


def _gap(got, ref):
    """tests/test_cuda.cpp:778-802: logits as maxErr, values as max-abs."""
    lg = O.max_err(got[0], ref[0])
    vg = float(np.abs(got[1].astype(np.float64) - ref[1]).max())
    return lg, vg


# (workload tag, batch checked against the oracle): the oracle's passes at
# these sizes take seconds.
PARITY_CASES = [(1, 8), (2, 64), (3, 8), (4, 1), (4, 8), (5, 1)]


@pytest.mark.parametrize("tag,B", PARITY_CASES)
def test_benchmark_workload_parity(hip, tag, B):
    """max-abs 1e-4 on logits and values against the blas
    restatement, argmax agreement >= 99.9%. Where the logits' size puts 1e-4
    below fp32 resolution (the 20x256 net's logits reach ~2.7e4, whose ulp is
    2e-3), the bar is the one the reference holds its GPU port to
    (tests/test_cuda.cpp:804-849): no further from blas than twice the
    reference's own naive backend is."""
    w = O.WORKLOADS[tag]
    net = O.init_network(w.cfg)
    inp, legal = O.workload_inputs(w, B)
    with _runner(hip, net, B) as r:
        got = r.infer(inp)
    blas = O.forward(net, inp, O.BLAS)
    naive = O.forward(net, inp, O.NAIVE)
    rep = parity_report(got[0], got[1], blas[0], blas[1], legal)
    cpu_l = float(np.abs(naive[0].astype(np.float64) - blas[0]).max())
    cpu_v = float(np.abs(naive[1].astype(np.float64) - blas[1]).max())
    rep.update(cpu_naive_vs_blas_logits=cpu_l, cpu_naive_vs_blas_values=cpu_v,
               max_abs_logit=float(np.abs(blas[0]).max()))
    print(f"workload {tag} B={B}: {rep}")
    assert np.isfinite(got[0]).all() and np.isfinite(got[1]).all()
    assert rep["logits_maxabs"] <= max(1e-4, 2 * cpu_l), rep
    assert rep["values_maxabs"] <= max(1e-4, 2 * cpu_v), rep
    assert rep["argmax_agree"] >= 0.999, rep
    if rep["max_abs_logit"] < 100:   # 1e-4 is above a few ulp of every logit
        assert rep["logits_maxabs"] <= 1e-4 and rep["values_maxabs"] <= 1e-4, rep
    if rep["max_abs_logit"] == 0:
        # Degenerate outputs (the 19x19 10x128 network with the synthetic BN
        # statistics: every policy pre-activation is negative, every logit the
        # zero bias, every value -1) show nothing of the trunk: compare it.
        with _runner(hip, net, B) as r:
            trunk = r.probe_trunk(inp, w.cfg.blocks)
        ref = O.trunk(net, inp, mode=O.BLAS)
        err = O.max_err(trunk, ref)
        print(f"workload {tag} B={B}: degenerate outputs; trunk maxErr {err:.3g} (max {ref.max():.4g})")
        assert ref.max() > 10 and err <= 1e-5, err


def test_wide_net_vs_double(hip):
    """The 20x256 net at batch 1 against the double-precision pass: the GPU's
    relative gap (maxErr) within max(1e-5, 2x the CPU backends' worst) and
    never above 5e-5 (tests/test_cuda.cpp:804-849)."""
    w = O.WORKLOADS[5]
    net = O.init_network(w.cfg)
    inp, _ = O.workload_inputs(w, 1)
    ref = O.forward_double(net, inp)
    with _runner(hip, net, 1) as r:
        g = _gap(r.infer(inp), ref)
    a = _gap(O.forward(net, inp, O.BLAS), ref)
    b = _gap(O.forward(net, inp, O.NAIVE), ref)
    print(f"wide net vs double: GPU {g}, blas {a}, naive {b}")
    for gg, cpu in zip(g, (max(a[0], b[0]), max(a[1], b[1]))):
        assert gg <= min(5e-5, max(1e-5, 2 * cpu)), (g, a, b)


@pytest.mark.parametrize("cfg,Bs", [
    (O.make_cfg(5, 3, 32), (1, 7, 16)),
    (O.make_cfg(9, 6, 64), (1, 7, 16)),
    (O.make_cfg(9, 2, 16, value_hidden=16), (1, 7)),
    (O.make_cfg(13, 6, 96), (1, 4)),
    (O.make_cfg(19, 10, 128, value_hidden=256), (1, 2)),
    (O.make_cfg(19, 2, 48), (3,)),
    (O.make_cfg(9, 0, 16), (5,)),
    # filters that leave the last 16-channel chunk or the last channel quad
    # part-filled, and input planes that fill whole chunks (history 7)
    (O.make_cfg(9, 2, 20), (1, 5)),
    (O.make_cfg(5, 2, 30, value_hidden=16), (3,)),
    (O.make_cfg(5, 1, 32, history=7), (2,)),
])
def test_random_networks_vs_double(hip, cfg, Bs):
    """tests/test_cuda.cpp:804-849 on random networks (random BN, biases):
    the GPU's gap to the double pass within max(1e-5, 2x the CPU backends'
    worst gap) and never above 5e-5."""
    net = O.random_network(cfg, 40 + cfg.board)
    rng = np.random.default_rng(611)
    with _runner(hip, net, max(Bs)) as r:
        for B in Bs:
            inp = rng.integers(0, 2, (B, cfg.planes, cfg.area)).astype(np.float32)
            ref = O.forward_double(net, inp)
            g = _gap(r.infer(inp), ref)
            a = _gap(O.forward(net, inp, O.BLAS), ref)
            b = _gap(O.forward(net, inp, O.NAIVE), ref)
            for gg, cpu in zip(g, (max(a[0], b[0]), max(a[1], b[1]))):
                assert gg <= min(5e-5, max(1e-5, 2 * cpu)), (cfg, B, g, a, b)


def test_headline_batch_independent(hip):
    """Workload 3 at its full batch of 256: a position's outputs are the same
    bits alone, at any slot of the full batch, and with the batch permuted
    (what the hub's determinism rests on, include/azgo/inference_hub.hpp:14-20)."""
    w = O.WORKLOADS[3]
    net = O.random_network(w.cfg, 602)
    inp, _ = O.workload_inputs(w, 256)
    with _runner(hip, net, 256) as r:
        whole = r.infer(inp)
        perm = np.random.default_rng(603).permutation(256)
        shuffled = r.infer(inp[perm])
        assert bitwise_equal(shuffled[0], whole[0][perm]) and bitwise_equal(shuffled[1], whole[1][perm])
        for s in (0, 1, 100, 255):
            alone = r.infer(inp[s:s + 1])
            assert bitwise_equal(alone[0][0], whole[0][s]) and bitwise_equal(alone[1][0], whole[1][s])
        for size in (8, 144):
            picks = np.random.default_rng(size).integers(0, 256, size)
            part = r.infer(inp[picks])
            assert bitwise_equal(part[0], whole[0][picks]) and bitwise_equal(part[1], whole[1][picks])


@pytest.mark.parametrize("B", [257, 75, 21, 17])
def test_split_pass_equals_whole(hip, B):
    """A batch with more than a round of workgroups, or a small one in the
    four-wave shape of 6 column groups, runs as two half-batch chains on two
    streams (forked and joined inside the captured graph), each half in its
    own batch's shape: an odd batch (257: whole-board workgroups; 75: the
    four-wave shape; 21: halves of 11 and 10 in a 2-group shape; 17: halves
    of 9 and 8 in two different shapes), captured and eager, gives every row
    the bits of the position alone, on both sides of the split."""
    w = O.WORKLOADS[3]
    net = O.random_network(w.cfg, 605)
    inp, _ = O.workload_inputs(w, B)
    half = (B + 1) // 2
    with _runner(hip, net, B) as r:
        graph = r.infer(inp)
        again = r.infer(inp)
        assert bitwise_equal(again[0], graph[0]) and bitwise_equal(again[1], graph[1])
        for s in (0, half - 2, half - 1, half, half + 1, B - 1):
            alone = r.infer(inp[s:s + 1])
            assert bitwise_equal(alone[0][0], graph[0][s]) and bitwise_equal(alone[1][0], graph[1][s])
        r.set_graphs(False)
        eager = r.infer(inp)
        assert bitwise_equal(eager[0], graph[0]) and bitwise_equal(eager[1], graph[1])
        ms, layers = r.time_tower_layers(0, B, 1)
        assert ms > 0 and layers == 2 * w.cfg.blocks


def test_every_batch_size_equals_singles(hip):
    """A runner at every batch size from 1 to 64 (tests/test_cuda.cpp:
    1022-1069 runs all of them): each size its own graph and workgroup
    shape, every row the bits of its position alone."""
    w = O.WORKLOADS[1]
    net = O.random_network(w.cfg, 606)
    inp, _ = O.workload_inputs(w, 64)
    with _runner(hip, net, 64, slots=2) as r:
        alone = [r.infer(inp[i:i + 1]) for i in range(64)]
        for B in range(1, 65):
            got = r.infer(inp[:B])
            for i in range(B):
                assert bitwise_equal(got[0][i], alone[i][0][0]) and bitwise_equal(got[1][i], alone[i][1][0]), (B, i)


def test_graph_cache_eviction_keeps_the_bits(hip):
    """A slot keeps at most 64 captured passes: 80 batch sizes in turn evict
    the least recently replayed ones, and a size captured again after its
    eviction (and one still cached) gives the same bits as before."""
    w = O.WORKLOADS[1]
    net = O.random_network(w.cfg, 608)
    inp, _ = O.workload_inputs(w, 80)
    with _runner(hip, net, 80, slots=1) as r:
        first = {B: r.infer(inp[:B]) for B in (1, 2, 3)}
        for B in range(4, 81):
            got = r.infer(inp[:B])
            assert np.isfinite(got[0]).all()
        for B in (1, 2, 3, 80):   # 1-3 were evicted, 80 is the newest
            again = r.infer(inp[:B])
            want = first.get(B, got)
            assert bitwise_equal(again[0], want[0]) and bitwise_equal(again[1], want[1]), B


@pytest.mark.parametrize("B", [5, 6, 8, 9, 16, 17, 18, 28, 29, 32, 33, 34, 115, 116, 128, 129, 217, 218])
def test_shape_and_split_boundaries(hip, B):
    """19x19 10x128 on both sides of each change of workgroup shape, of the
    two-chain split and of the halves' own shapes (17: halves of 9 and 8
    boards in two different shapes; 17-28 and 33: halves in a finer shape
    than the batch's): rows at the start, the middle and the end are the
    bits of their positions alone."""
    w = O.WORKLOADS[3]
    net = O.random_network(w.cfg, 607)
    inp, _ = O.workload_inputs(w, B)
    with _runner(hip, net, B) as r:
        whole = r.infer(inp)
        for s in (0, (B - 1) // 2, (B + 1) // 2, B - 1):
            alone = r.infer(inp[s:s + 1])
            assert bitwise_equal(alone[0][0], whole[0][s]) and bitwise_equal(alone[1][0], whole[1][s]), s


@pytest.mark.parametrize("tag,B", [(2, 128), (2, 129), (2, 191), (2, 192), (1, 1085), (1, 1086)])
def test_small_board_split_boundaries(hip, tag, B):
    """9x9 6x64 around the smaller shapes' split (two chains past two rounds
    of workgroups, from 129 boards) and the change to whole-board
    workgroups at 192 boards (one chain again); 5x5 4x32 around the least
    layer work that splits (0.5 GFLOP, from 1086 boards): rows on both
    sides of the halves are the bits of their positions alone."""
    w = O.WORKLOADS[tag]
    net = O.random_network(w.cfg, 608)
    inp, _ = O.workload_inputs(w, B)
    with _runner(hip, net, B) as r:
        whole = r.infer(inp)
        for s in (0, (B - 1) // 2, (B + 1) // 2, B - 1):
            alone = r.infer(inp[s:s + 1])
            assert bitwise_equal(alone[0][0], whole[0][s]) and bitwise_equal(alone[1][0], whole[1][s]), s


@pytest.mark.parametrize("cfg,B", [
    (O.make_cfg(5, 4, 32), 8),
    (O.make_cfg(5, 4, 32), 300),
    (O.make_cfg(5, 2, 30, value_hidden=16), 3),
    (O.make_cfg(5, 2, 16, ownership=1), 5),
    (O.make_cfg(5, 3, 64), 17),
    (O.make_cfg(9, 6, 64), 160),
    (O.make_cfg(9, 2, 56), 129),
    (O.make_cfg(9, 3, 32), 8),
    (O.make_cfg(9, 2, 20, value_hidden=16, ownership=1), 6),
    (O.make_cfg(13, 2, 16), 5),
    (O.make_cfg(13, 2, 32, value_hidden=256), 101),
    (O.make_cfg(5, 2, 32, history=1), 5),     # 4 input planes: one short chunk
    (O.make_cfg(9, 2, 32, history=7), 8),     # 16: one whole chunk, no short one
    (O.make_cfg(9, 2, 32, history=16), 9),    # 34: two whole chunks and 2 planes
])
def test_small_tower_equals_per_layer_launches(hip, cfg, B):
    """A small board's tower in one launch (one workgroup per board, the
    activations in LDS) gives the bits of the per-layer launches, graph and
    eager, including ragged channel counts and the ownership head."""
    net = O.random_network(cfg, 609)
    w = O.Workload(0, "small", cfg, B, 0.3, 0.3)
    inp, _ = O.workload_inputs(w, B)
    with _runner(hip, net, B) as r:
        one = r.infer(inp)
        r.set_small_tower(False)
        per_layer = r.infer(inp)
        r.set_graphs(False)
        eager = r.infer(inp)
        r.set_small_tower(True)
        one_eager = r.infer(inp)
    for got in (per_layer, eager, one_eager):
        assert len(got) == len(one)
        for a, b in zip(got, one):
            assert bitwise_equal(a, b)


@pytest.mark.parametrize("cfg,B", [
    (O.make_cfg(19, 10, 128), 256),   # the headline batch: the default takes it
    (O.make_cfg(19, 10, 128), 1),
    (O.make_cfg(19, 2, 128), 300),    # boards past the first round of workgroups
    (O.make_cfg(19, 2, 120, value_hidden=16, ownership=1), 5),   # a part-filled last block of channels
    (O.make_cfg(19, 1, 128, history=3), 3),    # 8 input planes: one short stem chunk
    (O.make_cfg(19, 1, 128, history=7), 2),    # 16: one whole chunk
    (O.make_cfg(19, 0, 128), 4),      # no residual blocks: the stem alone
])
def test_resident_tower_equals_per_layer_launches(hip, cfg, B):
    """A 19x19 pass with each board resident in one workgroup from the stem
    to the last layer gives the bits of the per-layer launches, graph and
    eager, with the heads (ownership included) after it."""
    net = O.random_network(cfg, 611)
    w = O.Workload(0, "resident", cfg, B, 0.3, 0.3)
    inp, _ = O.workload_inputs(w, B)
    with _runner(hip, net, B) as r:
        r.set_resident_tower(2)
        resident = r.infer(inp)
        r.set_resident_tower(0)
        per_layer = r.infer(inp)
        r.set_graphs(False)
        eager = r.infer(inp)
        r.set_resident_tower(2)
        resident_eager = r.infer(inp)
        r.set_resident_tower(1)
        default = r.infer(inp)
    for got in (per_layer, eager, resident_eager, default):
        assert len(got) == len(resident)
        for a, b in zip(got, resident):
            assert bitwise_equal(a, b)


def test_resident_tower_mode_refused(hip):
    net = O.random_network(O.make_cfg(5, 1, 16), 612)
    with _runner(hip, net, 2) as r:
        for bad in (-1, 3):
            with pytest.raises(hip.HipError):
                r.set_resident_tower(bad)
        with pytest.raises(hip.HipError):
            r.time_resident_tower(0, 2, 1)   # 5x5: not a network the resident tower takes


def test_pass_forms(hip):
    """How a pass runs, from the device's compute units (C): the
    board-resident tower for a pass alone whose batch gives one workgroup to
    95% of the CUs (one round) or to every CU in each of several rounds;
    otherwise, and beside another pass, the per-layer launches (on the
    MI355X's 256 CUs in half-batch chains there); the small-board pass in one
    launch on 9x9 at 64 channels past 128 boards."""
    cus = hip.device_cus()
    one_round = -(-19 * cus // 20)   # the fewest boards that give one workgroup to 95% of the CUs
    net = O.random_network(O.make_cfg(19, 2, 128), 613)
    with _runner(hip, net, 2 * cus) as r:
        assert r.pass_form(cus) == r.FORM_RESIDENT
        assert r.pass_form(one_round) == r.FORM_RESIDENT
        assert not r.pass_form(one_round - 1) & r.FORM_RESIDENT
        assert r.pass_form(2 * cus) == r.FORM_RESIDENT
        assert not r.pass_form(2 * cus - 8) & r.FORM_RESIDENT   # two rounds: only when full
        assert not r.pass_form(cus, alone=False) & r.FORM_RESIDENT
        assert r.pass_form(1) == 0
        if cus == 256:
            # The MI355X's measured forms beside them: two half-batch chains.
            assert r.pass_form(256, alone=False) == r.FORM_SPLIT
            assert r.pass_form(240) == r.FORM_SPLIT
            assert r.pass_form(504) == r.FORM_SPLIT
        r.set_resident_tower(2)
        assert r.pass_form(1) == r.FORM_RESIDENT and r.pass_form(cus, alone=False) == r.FORM_RESIDENT
        r.set_resident_tower(0)
        assert not r.pass_form(cus) & r.FORM_RESIDENT
        r.set_resident_tower(1)
        r.input(0)[:cus] = O.workload_inputs(O.Workload(0, "forms", net.cfg, cus, 0.3, 0.3), cus)[0]
        r.stage(0, cus)
        assert r.time_resident_tower(0, cus, 2) > 0 and r.time_resident_tower(0, cus, 2, stem=False) > 0
    net9 = O.random_network(O.make_cfg(9, 1, 64), 614)
    with _runner(hip, net9, 256) as r:
        assert r.pass_form(256) == r.FORM_SMALL


@pytest.mark.parametrize("history,B", [(8, 256), (7, 256), (9, 256), (16, 256), (8, 40), (3, 5)])
def test_input_plane_counts_parity(hip, history, B):
    """Networks of 2H + 2 input planes around the stem's chunking (18: a
    2-plane last chunk; 16: none; 20: 4 planes; 34: three chunks; 8: one
    short chunk), at 19x19 on the large-batch shapes (the stem in two halves
    of column groups) and smaller ones: logits within maxErr 5e-5 and values
    within 5e-5 of the oracle (the random-network bar above), and a board
    alone gives its bits in the batch."""
    cfg = O.make_cfg(19, 1, 128, history=history)
    net = O.random_network(cfg, 610 + history)
    w = O.Workload(0, "planes", cfg, B, 0.3, 0.3)
    inp, _ = O.workload_inputs(w, B)
    with _runner(hip, net, B) as r:
        got = r.infer(inp)
        alone = r.infer(inp[B - 1:B])
    ref = O.forward(net, inp, O.BLAS)
    assert O.max_err(got[0], ref[0]) <= 5e-5
    assert float(np.abs(got[1].astype(np.float64) - ref[1]).max()) <= 5e-5
    assert bitwise_equal(alone[0][0], got[0][B - 1]) and bitwise_equal(alone[1][0], got[1][B - 1])


@pytest.mark.parametrize("tag,B", [(4, 4), (4, 8), (4, 16), (2, 48), (2, 64), (5, 8)])
def test_alone_and_shared_shapes_same_bits(hip, tag, B):
    """A pass enqueued while the runner's other slot is idle takes the
    workgroup shapes fastest for one pass (one workgroup per CU); with a pass
    in flight on the other slot, the shapes that share the GPU better. The
    shape decides only which workgroup computes an output: the bits are the
    same either way, in both slots."""
    w = O.WORKLOADS[tag]
    net = O.random_network(w.cfg, 620 + tag)
    inp, _ = O.workload_inputs(w, B)
    with _runner(hip, net, B, slots=2) as r:
        alone = r.infer(inp)   # slot 0, slot 1 idle
        for slot in (0, 1):
            r.input(slot)[:B] = inp
        done = [threading.Event(), threading.Event()]
        errors = []

        def cb(slot, err):
            if err:
                errors.append(err)
            done[slot].set()

        hip.set_copy_out_delay(200000)   # each pass holds its slot for 0.2 s
        try:
            r.begin(1, B, cb)   # slot 0 idle: the shapes for one pass
            r.begin(0, B, cb)   # slot 1 busy: the shapes for two
            assert done[0].wait(60) and done[1].wait(60)
        finally:
            hip.set_copy_out_delay(0)
        assert not errors, errors
        for slot in (0, 1):
            assert bitwise_equal(r.logits(slot, B), alone[0]) and bitwise_equal(r.values(slot, B), alone[1]), slot


def test_repeatable_and_graph_equals_eager(hip):
    w = O.WORKLOADS[2]
    net = O.random_network(w.cfg, 604)
    inp, _ = O.workload_inputs(w, 32)
    with _runner(hip, net, 32) as r:
        first = r.infer(inp)
        for _ in range(5):
            again = r.infer(inp)
            assert bitwise_equal(again[0], first[0]) and bitwise_equal(again[1], first[1])
        r.set_graphs(False)
        eager = r.infer(inp)
        assert bitwise_equal(eager[0], first[0]) and bitwise_equal(eager[1], first[1])
    with _runner(hip, net, 32) as other:
        second = other.infer(inp)
        assert bitwise_equal(second[0], first[0])


def test_trunk_layers_vs_oracle(hip):
    """The trunk after the stem and after each block, against the naive
    restatement run to the same depth: maxErr per depth, growing slowly."""
    cfg = O.make_cfg(9, 3, 32)
    net = O.random_network(cfg, 71)
    inp = np.random.default_rng(72).integers(0, 2, (4, cfg.planes, cfg.area)).astype(np.float32)
    with _runner(hip, net, 4) as r:
        for depth in range(cfg.blocks + 1):
            got = r.probe_trunk(inp, depth)
            assert O.max_err(got, _double_trunk(net, inp, depth)) <= 1e-5, depth


def _double_trunk(net, inp, depth):
    """The trunk in float64 after the stem and `depth` blocks (the reference's forward)."""
    cfg = net.cfg
    t = {k: v.astype(np.float64) for k, v in net.tensors().items()}
    n, F = cfg.board, cfg.filters

    def conv(x, wname, cin, cout):
        B = x.shape[0]
        w = t[wname].reshape(cout, cin, 3, 3)
        xp = np.zeros((B, cin, n + 2, n + 2))
        xp[:, :, 1:-1, 1:-1] = x.reshape(B, cin, n, n)
        y = np.zeros((B, cout, n, n))
        for dy in range(3):
            for dx in range(3):
                y += np.einsum("oc,bcyx->boyx", w[:, :, dy, dx], xp[:, :, dy:dy + n, dx:dx + n])
        return y.reshape(B, cout, n * n)

    def bn(x, pre):
        scale = t[pre + ".gamma"] / np.sqrt(t[pre + ".runVar"] + np.float64(np.float32(1e-5)))
        return (x - t[pre + ".runMean"][None, :, None]) * scale[None, :, None] + t[pre + ".beta"][None, :, None]

    h = np.maximum(bn(conv(inp.astype(np.float64), "stem.conv.w", cfg.planes, F), "stem.bn"), 0)
    for i in range(depth):
        p = f"block{i}"
        m = np.maximum(bn(conv(h, p + ".conv1.w", F, F), p + ".bn1"), 0)
        h = np.maximum(bn(conv(m, p + ".conv2.w", F, F), p + ".bn2") + h, 0)
    return h


def test_heads_probe_vs_oracle(hip):
    """The heads kernel alone on a given trunk, against the heads of the
    double pass computed from the same trunk."""
    cfg = O.make_cfg(19, 1, 32)
    net = O.random_network(cfg, 81)
    rng = np.random.default_rng(82)
    trunk = rng.uniform(0, 2, (5, 32, 361)).astype(np.float32)
    with _runner(hip, net, 5) as r:
        logits, values = r.probe_heads(trunk)
    t = {k: v.astype(np.float64) for k, v in net.tensors().items()}
    x = trunk.astype(np.float64)

    def bn(v, pre, c):
        scale = t[pre + ".gamma"][c] / np.sqrt(t[pre + ".runVar"][c] + np.float64(np.float32(1e-5)))
        return (v - t[pre + ".runMean"][c]) * scale + t[pre + ".beta"][c]

    pw = t["policy.conv.w"].reshape(2, 32)
    pol = np.stack([np.maximum(bn(np.einsum("c,bcp->bp", pw[c], x), "policy.bn", c), 0) for c in range(2)], 1)
    ref_logits = pol.reshape(5, -1) @ t["policy.fc.w"].reshape(362, 722).T + t["policy.fc.b"]
    val = np.maximum(bn(np.einsum("c,bcp->bp", t["value.conv.w"], x), "value.bn", 0), 0)
    hid = np.maximum(val @ t["value.fc1.w"].reshape(64, 361).T + t["value.fc1.b"], 0)
    ref_values = np.tanh(hid @ t["value.fc2.w"] + t["value.fc2.b"][0])
    assert O.max_err(logits, ref_logits) <= 1e-5
    assert np.abs(values - ref_values).max() <= 1e-5


@pytest.mark.parametrize("cfg,B", [
    (O.make_cfg(5, 2, 32, ownership=1), 8),
    (O.make_cfg(9, 2, 16, 8, ownership=1), 7),
    (O.make_cfg(19, 2, 48, ownership=1), 4),
])
def test_ownership_head_vs_oracle(hip, cfg, B):
    """The ownership head (src/network.cpp:298-308: 1x1 conv F -> 1, BN, tanh
    at every point) through CudaInference::infer's contract: against the
    blas restatement (1e-4) and the double pass (within twice the CPU's own
    gap); the same pass's logits and values are bit for bit those of the
    network without the head, and asking a network without it for ownership
    is an argument error (src/cuda/cuda_network.cu:316)."""
    net = O.random_network(cfg, 90 + cfg.board)
    rng = np.random.default_rng(91)
    inp = rng.integers(0, 2, (B, cfg.planes, cfg.area)).astype(np.float32)
    with _runner(hip, net, B) as r:
        logits, values, own = r.infer(inp, ownership=True)
        again = r.infer(inp)
    blas = O.forward(net, inp, O.BLAS, ownership=True)
    dbl = O.forward_double(net, inp, ownership=True)
    gpu_gap = float(np.abs(own.astype(np.float64) - dbl[2]).max())
    cpu_gap = float(np.abs(blas[2].astype(np.float64) - dbl[2]).max())
    print(f"{cfg}: ownership gap to double {gpu_gap:.3g} (blas {cpu_gap:.3g})")
    assert own.shape == (B, cfg.area) and np.isfinite(own).all()
    assert float(np.abs(own - blas[2]).max()) <= 1e-4
    assert gpu_gap <= max(1e-5, 2 * cpu_gap)
    assert bitwise_equal(again[0], logits) and bitwise_equal(again[1], values)
    plain = O.make_cfg(cfg.board, cfg.blocks, cfg.filters, cfg.value_hidden)
    tensors = {k: v for k, v in net.tensors().items() if not k.startswith("ownership.")}
    with hip.Runner(to_hip_cfg(hip, plain), tensors, B) as r:
        base = r.infer(inp)
        with pytest.raises(hip.HipError) as e:
            r.infer(inp, ownership=True)
        assert e.value.code == hip.ERR_ARGUMENT
    assert bitwise_equal(base[0], logits) and bitwise_equal(base[1], values)


def test_ownership_heads_probe_vs_double(hip):
    """The heads kernels alone with the ownership head on a given trunk:
    tanh(bn(w . x)) per point against float64."""
    cfg = O.make_cfg(19, 1, 32, ownership=1)
    net = O.random_network(cfg, 83)
    trunk = np.random.default_rng(84).uniform(0, 2, (3, 32, 361)).astype(np.float32)
    with _runner(hip, net, 3) as r:
        _, _, own = r.probe_heads(trunk, ownership=True)
    t = {k: v.astype(np.float64) for k, v in net.tensors().items()}
    conv = np.einsum("c,bcp->bp", t["ownership.conv.w"], trunk.astype(np.float64))
    scale = t["ownership.bn.gamma"][0] / np.sqrt(t["ownership.bn.runVar"][0] + np.float64(np.float32(1e-5)))
    ref = np.tanh((conv - t["ownership.bn.runMean"][0]) * scale + t["ownership.bn.beta"][0])
    assert float(np.abs(own - ref).max()) <= 1e-5


def test_tanh_within_two_ulp(hip):
    """The heads' tanh (value and ownership, tanhf) within 2 ulp of tanh in
    double (tests/test_cuda.cpp:494-512). The ownership head is made to pass
    a trunk value straight through: 1x1 weights selecting channel 0 (the
    other channels' terms add exact zeros), BN with gamma 1, beta 0, mean 0
    and a variance whose float sum with eps is exactly 1."""
    cfg = O.make_cfg(9, 1, 16, ownership=1)
    net = O.random_network(cfg, 85)
    t = net.tensors()
    t["ownership.conv.w"][:] = 0.0
    t["ownership.conv.w"][0] = 1.0
    t["ownership.bn.gamma"][:] = 1.0
    t["ownership.bn.beta"][:] = 0.0
    t["ownership.bn.runMean"][:] = 0.0
    t["ownership.bn.runVar"][:] = np.float32(0.99999)
    assert np.float32(0.99999) + np.float32(1e-5) == np.float32(1.0)
    B = 8
    rng = np.random.default_rng(86)
    trunk = rng.uniform(-1, 1, (B, 16, 81)).astype(np.float32)
    x = np.concatenate([np.linspace(-9.5, 9.5, 400), rng.uniform(-3, 3, 200),
                        [1e-7, -1e-7, 1e-20, 3e-4, -3e-4, 0.5493, 0.881, 20.0, -20.0, 1e-3, 0.1, -0.1, 2.0, 5.0,
                         8.6, 9.1, 0.03, 0.7, -0.7, 1.5, 4.0, 0.25, 0.125, 0.0625, 1.0, -1.0, 3.0, 0.9]]).astype(np.float32)
    x = x[:B * 81]
    x = np.concatenate([x, np.full(B * 81 - len(x), 0.375, np.float32)])
    trunk[:, 0, :] = x.reshape(B, 81)
    with hip.Runner(to_hip_cfg(hip, cfg), t, B, 1) as r:
        _, _, own = r.probe_heads(trunk, ownership=True)
    ref = np.tanh(x.astype(np.float64))
    got = own.reshape(-1).astype(np.float64)
    ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    err = np.abs(got - ref) / ulp
    assert float(err.max()) <= 2.0, (float(err.max()), float(x[np.argmax(err)]))


def test_runner_threads_released(hip):
    """No thread outlives its runner (tests/test_cuda.cpp:1220-1237): the
    process's thread count after creating, using and destroying runners of
    one and two slots is what it was before."""
    w = O.WORKLOADS[1]
    net = O.init_network(w.cfg)
    inp, _ = O.workload_inputs(w, 8)
    count = lambda: len(os.listdir("/proc/self/task"))
    with _runner(hip, net, 8, slots=2) as r:   # the HIP runtime's own threads start here
        r.infer(inp)
    before = count()
    for slots in (1, 2, 1, 2):
        with _runner(hip, net, 8, slots=slots) as r:
            r.infer(inp)
            for s in range(slots):
                r.input(s)[:8] = inp
            r.time_pipelined(8, 6)
    assert count() == before


def test_softmax_legal_vs_oracle(hip):
    """Mcts::expand's priors (src/mcts.cpp:170-183), restated in the oracle."""
    w = O.WORKLOADS[3]
    rng = np.random.default_rng(5)
    B = 64
    logits = (rng.standard_normal((B, 362)) * 20).astype(np.float32)
    _, legal = O.workload_inputs(w, B)
    legal[3, :] = 0
    legal[3, 361] = 1   # only pass legal
    got = hip.softmax_legal(logits, legal)
    ref = O.softmax_legal(logits, legal)
    assert np.all(got[legal == 0] == 0)
    assert np.abs(got.astype(np.float64) - ref).max() <= 1e-6
    ok = ref > 1e-30
    assert (np.abs(got[ok].astype(np.float64) - ref[ok]) <= 4e-6 * ref[ok]).all()
    assert np.allclose(got.sum(axis=1), 1.0, atol=1e-5)
    assert got[3, 361] == 1.0


def test_softmax_register_and_loop_kernels_agree(hip):
    """Rows of up to 384 actions take the register kernel, longer ones the
    loop kernel; with one more action that is illegal both sum the same
    values in the same order, so the priors are the same bits."""
    rng = np.random.default_rng(9)
    B, A = 37, 384
    logits = (rng.standard_normal((B, A)) * 8).astype(np.float32)
    legal = (rng.random((B, A)) < 0.6).astype(np.uint8)
    legal[5, :] = 0   # nothing legal: all zeros
    regs = hip.softmax_legal(logits, legal)
    longer = hip.softmax_legal(np.concatenate([logits, np.full((B, 1), 50.0, np.float32)], axis=1),
                               np.concatenate([legal, np.zeros((B, 1), np.uint8)], axis=1))
    assert bitwise_equal(regs, longer[:, :A]) and np.all(longer[:, A] == 0)
    assert np.all(regs[5] == 0)
    ref = O.softmax_legal(logits, legal)
    assert np.abs(regs.astype(np.float64) - ref).max() <= 1e-6


def test_runner_slots_async(hip):
    """BatchRunner's contract (include/azgo/inference_hub.hpp:41-53): begin on
    each slot returns at once, done comes once per pass from the completion
    thread, and the slot's outputs equal the synchronous pass bit for bit;
    the copy-out delay hook proves done waits for the outputs
    (tests/test_cuda.cpp:1076-1091)."""
    w = O.WORKLOADS[2]
    net = O.init_network(w.cfg)
    inp, _ = O.workload_inputs(w, 64)
    with _runner(hip, net, 64, slots=2) as r:
        sync = r.infer(inp[:40])
        before = hip.passes_completed()
        for delay in (0, 20000):
            hip.set_copy_out_delay(delay)
            events = [threading.Event(), threading.Event()]
            errors = [None, None]

            def done(slot, err):
                errors[slot] = err
                events[slot].set()

            for slot, B in ((0, 40), (1, 17)):
                r.input(slot)[:B] = inp[:B]
                r.begin(slot, B, done)
            for e in events:
                assert e.wait(30)
            hip.set_copy_out_delay(0)
            assert errors == [None, None]
            assert bitwise_equal(r.logits(0, 40), sync[0]) and bitwise_equal(r.values(0, 40), sync[1])
            assert bitwise_equal(r.logits(1, 17), sync[0][:17])
        assert hip.passes_completed() - before == 4


def test_runner_failure_injection(hip):
    """cuda_probe::failPassesAfter (src/cuda/cuda_runner.cu:175-179): after n
    normal passes the next reports a failure through done, once."""
    w = O.WORKLOADS[1]
    net = O.init_network(w.cfg)
    inp, _ = O.workload_inputs(w, 8)
    with _runner(hip, net, 8, slots=1) as r:
        r.input(0)[:8] = inp
        hip.fail_passes_after(2)
        results = []
        for _ in range(4):
            ev = threading.Event()
            r.begin(0, 8, lambda s, e: (results.append(e), ev.set()))
            assert ev.wait(30)
        hip.fail_passes_after(0)
        assert results[0] is None and results[1] is None and results[3] is None
        assert results[2] and "injected failure" in results[2]


def test_runner_kept_full(hip):
    """The reference bench's pipelined measurement (apps/bench.cpp:227-279)
    through begin/done: every pass completes once, each slot's outputs are
    the synchronous pass's bits, and an injected failure stops the
    resubmission, drains the passes in flight and is reported."""
    w = O.WORKLOADS[2]
    net = O.init_network(w.cfg)
    inp, _ = O.workload_inputs(w, 64)
    with _runner(hip, net, 64, slots=2) as r:
        sync = r.infer(inp[:48])
        for slot in (0, 1):
            r.input(slot)[:48] = inp[:48]
        before = hip.passes_completed()
        ms = r.time_pipelined(48, 9)
        assert ms > 0 and hip.passes_completed() - before == 9
        for slot in (0, 1):
            assert bitwise_equal(r.logits(slot, 48), sync[0]) and bitwise_equal(r.values(slot, 48), sync[1])
        hip.fail_passes_after(3)
        try:
            with pytest.raises(hip.HipError, match="injected failure"):
                r.time_pipelined(48, 20)
        finally:
            hip.fail_passes_after(0)
        # Drained: both slots take passes again.
        assert r.time_pipelined(48, 2) > 0


def test_runner_rejects_bad_begin(hip):
    w = O.WORKLOADS[1]
    net = O.init_network(w.cfg)
    with _runner(hip, net, 8, slots=1) as r:
        for slot, B in ((0, 0), (0, 9), (1, 4)):
            with pytest.raises(hip.HipError) as e:
                r.begin(slot, B, lambda s, err: None)
            assert e.value.code == hip.ERR_ARGUMENT


def test_busy_slot_refusal_keeps_the_pass_in_flight(hip):
    """A begin on a slot whose pass is still in flight (held by the copy-out
    delay) is refused with a state error and calls nothing, and so is a
    synchronous call on that slot; the first pass's done still comes exactly
    once, with the synchronous pass's bits."""
    w = O.WORKLOADS[1]
    net = O.init_network(w.cfg)
    inp, _ = O.workload_inputs(w, 8)
    with _runner(hip, net, 8, slots=1) as r:
        sync = r.infer(inp)
        r.input(0)[:8] = inp
        calls = []
        ev = threading.Event()
        hip.set_copy_out_delay(200000)
        try:
            r.begin(0, 8, lambda s, e: (calls.append(e), ev.set()))
            with pytest.raises(hip.HipError) as e1:
                r.begin(0, 8, lambda s, e: calls.append("second"))
            with pytest.raises(hip.HipError) as e2:
                r.infer(inp)
        finally:
            hip.set_copy_out_delay(0)
        assert e1.value.code == hip.ERR_STATE and e2.value.code == hip.ERR_STATE
        assert ev.wait(30)
        time.sleep(0.05)
        assert calls == [None]
        assert bitwise_equal(r.logits(0, 8), sync[0]) and bitwise_equal(r.values(0, 8), sync[1])


def test_memory_check_groups(hip):
    """checkCudaInferenceMemory's overload over GpuHubs groups
    (src/cuda/cuda_runner.cu:242-256): the groups are summed, the refusal
    names every hub and the largest batch, and the sum of two groups equals
    the memory of their runners."""
    cfg = to_hip_cfg(hip, O.WORKLOADS[3].cfg)
    hip.set_memory_limit(1 << 20)
    try:
        with pytest.raises(hip.HipError) as e:
            hip.check_memory_groups(cfg, [(1, 2, 256), (2, 1, 64)])
        msg = str(e.value)
        assert e.value.code == hip.ERR_MEMORY and "(3 hubs)" in msg and "inference_batch 256" in msg
        need = hip.memory_need(cfg, 256, 2) + 2 * hip.memory_need(cfg, 64, 1)
        assert f"needs {need // 10**6} MB" in msg
        hip.set_memory_limit(need)
        hip.check_memory_groups(cfg, [(1, 2, 256), (2, 1, 64)])   # exactly fits
        hip.set_memory_limit(need - 1)
        with pytest.raises(hip.HipError):
            hip.check_memory_groups(cfg, [(1, 2, 256), (2, 1, 64)])
    finally:
        hip.set_memory_limit(0)


def test_memory_check_message(hip):
    """checkFits's refusal (src/cuda/cuda_runner.cu:206-223) through the
    stand-in memory limit."""
    cfg = to_hip_cfg(hip, O.WORKLOADS[3].cfg)
    hip.set_memory_limit(10 << 20)
    try:
        with pytest.raises(hip.HipError) as e:
            hip.check_memory(cfg, 256, 1, 2)
        assert e.value.code == hip.ERR_MEMORY and str(e.value).endswith("lower inference_batch")
    finally:
        hip.set_memory_limit(0)
    hip.check_memory(cfg, 256, 1, 2)


def test_fill_probe_tail_untouched(hip):
    data = np.arange(20, dtype=np.float32)
    out = hip.probe_fill(data, 16, 2.5, tail=4)
    assert np.all(out[:16] == 2.5) and np.array_equal(out[16:], data[16:])


def test_mfma_probe(hip):
    """The matrix-rate probe: one 8-wave workgroup per CU (256 on the
    MI355X), each wave 4 x chain MFMAs of 2048 flops, at a rate no higher
    than the published 157.3 TFLOP/s peak and not far below it."""
    ms, flops = hip.probe_mfma(2000, 2)
    assert flops == hip.device_cus() * 8 * 4 * 2000 * 2048
    tf = flops / (ms / 2 * 1e-3) / 1e12
    assert 100.0 < tf <= 157.3 * 1.01, tf
    with pytest.raises(hip.HipError):
        hip.probe_mfma(0, 1)


def test_describe(hip):
    d = hip.describe()
    assert "gfx950" in d and "kernels" in d
