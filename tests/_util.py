"""Shared helpers of the tests (not collected: the name starts with _)."""
import os

import numpy as np

import oracle as O

U = 2.0 ** -24   # fp32 unit roundoff


def board_to_channel(x):
    """[B][C][A] -> [C][B*A] (the reference's channel-major activations)."""
    B, Cc, A = x.shape
    return np.ascontiguousarray(x.transpose(1, 0, 2)).reshape(Cc, B * A)


def channel_to_board(y, B):
    Cc = y.shape[0]
    return np.ascontiguousarray(y.reshape(Cc, B, -1).transpose(1, 0, 2))


def oracle_conv_raw(x, w):
    """The reference's im2col + naive gemm on [B][cin][A] input -> [B][cout][A]."""
    B, cin, A = x.shape
    n = int(round(A ** 0.5))
    cout = w.shape[0]
    y = O.conv3x3(w, cin, cout, board_to_channel(x), B, n, O.NAIVE)
    return channel_to_board(y.reshape(cout, B * A), B)


def conv_exact_and_bound(x, w):
    """The 3x3 'same' convolution in float64 and sum|w||x| per output:
    any fp32 evaluation order lands within K * u * sum|w||x| of the exact sum."""
    B, cin, A = x.shape
    n = int(round(A ** 0.5))
    cout = w.shape[0]
    xd = x.astype(np.float64).reshape(B, cin, n, n)
    wd = w.astype(np.float64).reshape(cout, cin, 3, 3)
    pad = np.zeros((B, cin, n + 2, n + 2))
    pad[:, :, 1:-1, 1:-1] = xd
    exact = np.zeros((B, cout, n, n))
    mag = np.zeros((B, cout, n, n))
    for dy in range(3):
        for dx in range(3):
            patch = pad[:, :, dy:dy + n, dx:dx + n]
            exact += np.einsum("oc,bcyx->boyx", wd[:, :, dy, dx], patch)
            mag += np.einsum("oc,bcyx->boyx", np.abs(wd[:, :, dy, dx]), np.abs(patch))
    return exact.reshape(B, cout, A), mag.reshape(B, cout, A)


def epilogue_f32(acc, scale, shift, skip, relu):
    """scale * acc + shift (+ skip), ReLU, each operation rounded in float32."""
    s = np.asarray(scale, np.float32)[None, :, None]
    h = np.asarray(shift, np.float32)[None, :, None]
    v = (s * acc.astype(np.float32)).astype(np.float32) + h
    if skip is not None:
        v = v + skip.astype(np.float32)
    if relu:
        v = np.where(v > 0, v, np.float32(0))
    return v.astype(np.float32)


def bitwise_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def to_hip_cfg(hip, cfg):
    return hip.net_cfg(cfg.board, cfg.history, cfg.blocks, cfg.filters, cfg.value_hidden, cfg.ownership)


def parity_report(got_logits, got_values, ref_logits, ref_values, legal=None):
    d = {
        "logits_maxabs": float(np.abs(got_logits.astype(np.float64) - ref_logits).max()),
        "logits_maxerr": float(O.max_err(got_logits, ref_logits)),
        "values_maxabs": float(np.abs(got_values.astype(np.float64) - ref_values).max()),
    }
    if legal is not None:
        d["argmax_agree"] = float((O.legal_argmax(got_logits, legal) == O.legal_argmax(ref_logits, legal)).mean())
    return d


GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def calibrated_network(tag, cfg=None):
    """Generation 0 as the reference's trainer makes it: Network(cfg, 1)'s
    weights (the oracle's init, pinned bitwise to the reference) with the
    batch-norm running statistics the reference's calibrateBatchNorm wrote
    (tests/golden/calibrated_bn.npz, key prefix `tag`)."""
    if cfg is None:
        cfg = O.WORKLOADS[int(tag)].cfg
    net = O.init_network(cfg, synthetic_bn=False)
    with np.load(os.path.join(GOLDEN, "calibrated_bn.npz")) as z:
        found = 0
        for name, t in net.tensors().items():
            key = f"{tag}/{name}"
            if key in z:
                t[:] = z[key]
                found += 1
    assert found == 2 * (2 * cfg.blocks + 3 + (1 if cfg.ownership else 0)), found
    return net
