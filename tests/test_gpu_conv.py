"""The fused 3x3 convolution kernel (stem and residual tower) on the GPU
against the oracle: the reference's im2col + gemm (src/backend.cpp:21-55,
src/layers.cpp:35-46) followed by BatchNorm2d::forwardInfer's arithmetic
(src/layers.cpp:88-97), the skip add and ReLU (src/network.cpp:264-271).

What the tests pin:
- every output within the fp32 summation bound K * u * sum|w||x| of the exact
  (float64) convolution, and maxErr <= 1e-5 against the oracle (the ceiling of
  tests/test_cuda.cpp:756-776);
- the fused epilogue equals the kernel's raw sums pushed through the
  reference's BN/skip/ReLU roundings, bit for bit (tests/test_cuda.cpp:570-596);
- outputs bitwise independent of the workgroup tiling and of the batch
  (tests/test_cuda.cpp:340-374, 600-623);
- zero halo: a board's edge sees zeros, never a neighbour's points.
"""
import numpy as np
import pytest

import build
import oracle as O
from _util import (U, bitwise_equal, conv_exact_and_bound, epilogue_f32, oracle_conv_raw)

pytestmark = pytest.mark.gpu

TILINGS = build.conv_tiling_count()   # the workgroup shapes the kernel is built for

SHAPES = [  # (n, cin, cout, B): stem and tower shapes of the five workloads, plus ragged ones
    (5, 18, 32, 3), (5, 32, 32, 8), (9, 18, 64, 2), (9, 64, 64, 5), (19, 18, 128, 2), (19, 128, 128, 3),
    (19, 256, 256, 1), (13, 40, 24, 2), (19, 7, 20, 2), (9, 32, 30, 3), (5, 16, 18, 2),
]


def _rand(rng, *shape, lo=-1.0, hi=1.0):
    return rng.uniform(lo, hi, shape).astype(np.float32)


@pytest.mark.parametrize("n,cin,cout,B", SHAPES)
def test_conv_within_fp32_bound_and_maxerr(hip, n, cin, cout, B):
    rng = np.random.default_rng(1000 + n * 7 + cin + cout)
    A = n * n
    x = _rand(rng, B, cin, A)
    w = (rng.standard_normal((cout, cin * 9)) * np.sqrt(2.0 / (cin * 9))).astype(np.float32)
    ones, zeros = np.ones(cout, np.float32), np.zeros(cout, np.float32)
    got = hip.probe_conv3x3(x, w, ones, zeros, relu=False)
    exact, mag = conv_exact_and_bound(x, w)
    K = cin * 9
    err = np.abs(got.astype(np.float64) - exact)
    assert (err <= K * U * mag + 1e-30).all(), f"worst {(err / (K * U * mag + 1e-30)).max():.2f} of the bound"
    ref = oracle_conv_raw(x, w)
    assert O.max_err(got, ref) <= 1e-5


@pytest.mark.parametrize("n,cin,cout,B", [(19, 128, 128, 2), (9, 64, 64, 3), (5, 18, 32, 2)])
def test_fused_epilogue_equals_explicit(hip, n, cin, cout, B):
    rng = np.random.default_rng(77 + n)
    A = n * n
    x = _rand(rng, B, cin, A)
    w = _rand(rng, cout, cin * 9, lo=-0.1, hi=0.1)
    scale = _rand(rng, cout, lo=0.5, hi=2.0)
    shift = _rand(rng, cout, lo=-0.5, hi=0.5)
    skip = _rand(rng, B, cout, A)
    raw = hip.probe_conv3x3(x, w, np.ones(cout, np.float32), np.zeros(cout, np.float32), relu=False)
    for sk in (None, skip):
        for relu in (False, True):
            fused = hip.probe_conv3x3(x, w, scale, shift, skip=sk, relu=relu)
            assert bitwise_equal(fused, epilogue_f32(raw, scale, shift, sk, relu))


@pytest.mark.parametrize("n,cin,cout", [(19, 128, 128), (9, 64, 64), (19, 18, 128)])
def test_tilings_bitwise_identical(hip, n, cin, cout):
    rng = np.random.default_rng(5)
    x = _rand(rng, 3, cin, n * n)
    w = _rand(rng, cout, cin * 9, lo=-0.1, hi=0.1)
    s, h = _rand(rng, cout), _rand(rng, cout)
    outs = [hip.probe_conv3x3(x, w, s, h, relu=True, tiling=t) for t in range(TILINGS)]
    for o in outs[1:]:
        assert bitwise_equal(o, outs[0])


@pytest.mark.parametrize("cin", [2, 4, 5, 16, 18, 20, 30, 34])
def test_stem_last_chunk_every_tiling(hip, cin):
    """The stem's input planes (cin not a multiple of 16 leaves a short last
    chunk, whose (plane, tap) pairs run packed four to an MFMA: straight-line
    for 2 planes, a step at a time otherwise; cin <= 32 on whole boards runs
    in two halves of column groups): every tiling gives the same bits, within
    the fp32 summation bound and maxErr <= 1e-5 of the oracle."""
    rng = np.random.default_rng(300 + cin)
    n, cout, B = 19, 128, 3
    x = _rand(rng, B, cin, n * n)
    w = (rng.standard_normal((cout, cin * 9)) * np.sqrt(2.0 / (cin * 9))).astype(np.float32)
    ones, zeros = np.ones(cout, np.float32), np.zeros(cout, np.float32)
    outs = [hip.probe_conv3x3(x, w, ones, zeros, relu=False, tiling=t) for t in range(TILINGS)]
    for o in outs[1:]:
        assert bitwise_equal(o, outs[0])
    exact, mag = conv_exact_and_bound(x, w)
    err = np.abs(outs[0].astype(np.float64) - exact)
    assert (err <= cin * 9 * U * mag + 1e-30).all()
    assert O.max_err(outs[0], oracle_conv_raw(x, w)) <= 1e-5


@pytest.mark.parametrize("tiling", [1, 4, 8])
def test_stem_with_skip_every_body(hip, tiling):
    """Input planes with a residual (not the network's stem, which adds
    nothing, but the probe's contract): whole-board shapes run the one-pass
    body then, and the fused epilogue still equals the explicit one."""
    rng = np.random.default_rng(81)
    n, cin, cout, B = 19, 18, 128, 2
    x = _rand(rng, B, cin, n * n)
    w = _rand(rng, cout, cin * 9, lo=-0.1, hi=0.1)
    scale = _rand(rng, cout, lo=0.5, hi=2.0)
    shift = _rand(rng, cout, lo=-0.5, hi=0.5)
    skip = _rand(rng, B, cout, n * n)
    raw = hip.probe_conv3x3(x, w, np.ones(cout, np.float32), np.zeros(cout, np.float32), relu=False,
                            tiling=tiling)
    fused = hip.probe_conv3x3(x, w, scale, shift, skip=skip, relu=True, tiling=tiling)
    assert bitwise_equal(fused, epilogue_f32(raw, scale, shift, skip, True))


def test_conv_batch_independent(hip):
    rng = np.random.default_rng(9)
    n, cin, cout = 19, 128, 128
    pool = _rand(rng, 40, cin, n * n)
    w = _rand(rng, cout, cin * 9, lo=-0.1, hi=0.1)
    s, h = _rand(rng, cout), _rand(rng, cout)
    whole = hip.probe_conv3x3(pool, w, s, h, relu=True)
    for i in (0, 1, 17, 39):
        alone = hip.probe_conv3x3(pool[i:i + 1], w, s, h, relu=True)
        assert bitwise_equal(whole[i], alone[0])
    perm = rng.permutation(40)
    shuffled = hip.probe_conv3x3(pool[perm], w, s, h, relu=True)
    assert bitwise_equal(shuffled, whole[perm])


def test_zero_halo_no_neighbour_leak(hip):
    """A lone board of ones beside boards of huge values: its outputs are the
    hand-countable neighbourhood sizes (4 corners, 6 edges, 9 inside with an
    all-ones kernel), untouched by its neighbours."""
    n, cin, cout = 19, 16, 16
    x = np.full((3, cin, n * n), 1e6, np.float32)
    x[1] = 1.0
    w = np.zeros((cout, cin * 9), np.float32)
    w[:, :9] = 1.0   # input channel 0, every tap
    got = hip.probe_conv3x3(x, w, np.ones(cout, np.float32), np.zeros(cout, np.float32), relu=False)
    counts = np.full((n, n), 9.0)
    counts[0, :] = counts[-1, :] = counts[:, 0] = counts[:, -1] = 6.0
    counts[0, 0] = counts[0, -1] = counts[-1, 0] = counts[-1, -1] = 4.0
    for co in range(cout):
        assert np.array_equal(got[1, co].reshape(n, n), counts)


def test_conv_hand_example(hip):
    """tests/test_layers.cpp:145-157: an all-ones 3x3 kernel on 1..9 (n = 3 is
    not a supported board, so the 3x3 image sits in a corner of a 5x5 board of
    zeros, which the zero padding makes equivalent for its own points)."""
    n = 5
    x = np.zeros((1, 1, n * n), np.float32)
    img = np.arange(1, 10, dtype=np.float32).reshape(3, 3)
    xb = x.reshape(1, 1, n, n)
    xb[0, 0, :3, :3] = img
    w = np.ones((1, 9), np.float32)
    got = hip.probe_conv3x3(x, w, np.ones(1, np.float32), np.zeros(1, np.float32), relu=False).reshape(n, n)
    # Points (0..1, 0..1) see only the image; compare those with the hand values.
    expected = np.array([12, 21, 16, 27, 45, 33, 24, 39, 28], np.float32).reshape(3, 3)
    assert np.array_equal(got[:2, :2], expected[:2, :2])


def test_relu_special_values(hip):
    """ReLU maps -0 and NaN to +0 (reluForward, src/layers.cpp:191-195;
    tests/test_cuda.cpp:468-490): shift = -0 with a zero input, and NaN inputs."""
    n, cin, cout = 5, 16, 16
    x = np.zeros((1, cin, n * n), np.float32)
    w = np.zeros((cout, cin * 9), np.float32)
    s = np.ones(cout, np.float32)
    h = np.full(cout, -0.0, np.float32)
    got = hip.probe_conv3x3(x, w, s, h, relu=True)
    assert np.all(got.view(np.uint32) == 0)
    x[0, 0, 12] = np.nan
    w[:, 4] = 1.0   # centre tap of channel 0
    got = hip.probe_conv3x3(x, w, s, np.zeros(cout, np.float32), relu=True)
    assert got[0, :, 12].view(np.uint32).tolist() == [0] * cout
