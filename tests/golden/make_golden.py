"""Writes the golden vectors under tests/golden/ from the REFERENCE's own code:
its sources compiled in place into oracle/_ref/libazgo_ref.so by
oracle/Makefile (naive backend; the reference's BLAS backend needs
<cblas.h>, which this image lacks). Run where the reference tree is present:

    make -C oracle && python tests/golden/make_golden.py

Vectors (data only, no reference source):
  rng.json        Rng(seed).next()/uniform()/normal()/below() draws and
                  deriveSeed values (src/rng.cpp)
  weights.json    sha256 of every tensor of Network(cfg, 1) for the five
                  workloads' shapes (src/network.cpp:77-111), params() order
  encode.npz      encodePlanes outputs (src/encode.cpp:14-43) for fixed
                  stone patterns under all 8 symmetries
  infer_*.npz     Network::infer (naive backend) inputs and outputs: the
                  5x5 4x32 workload (seeded weights, synthetic BN statistics,
                  batch 8) and a 9x9 2x16 network with random BN and biases
  calibrated_bn.npz  generation 0's batch-norm running statistics: every
                  runMean/runVar of Network(cfg, 1) after calibrateBatchNorm
                  (src/bn_calibration.cpp:33-45) with the trainer's seed
                  deriveSeed(1, 0, 7) (src/trainer.cpp:559), for the five
                  workloads' shapes and the 19x19 preset's value head of 256
  gen0_*.azn      checkpoints written by saveNetwork (src/checkpoint.cpp:84-100):
                  calibrated generation 0 of the 5x5 4x32 workload network
                  (version 1) and of a 5x5 2x16 network with the ownership
                  head (version 2)
  gen0_infer.npz  Network::infer of those two checkpoints as loadNetwork
                  reads them, on the 5x5 workload's batch of 8 positions
  trunk.npz       the trunk (stem and the first k residual blocks,
                  src/network.cpp:241-272) of the reference's Network::infer,
                  read out through its own policy head made an exact copy:
                  a one-hot 1x1 conv row picks channel c, the batch norm is
                  the identity (gamma 1, beta 0, mean 0, runVar 1 - 1e-5,
                  whose scale rounds to exactly 1), the ReLU passes the
                  trunk's nonnegative values, and an identity Linear with
                  zero bias copies the A points into the first A logits; for
                  the 5x5 4x32 workload network (k = 0, 2, 4) and a 9x9 2x16
                  network with random BN and biases (k = 2)
  games.npz       random games played by the reference's Game with
                  bnCalibrationPositions' move choice (src/bn_calibration.cpp:19-28):
                  every position's stones, side to move, Board::hash and the
                  legal set Mcts::expand builds at a root (src/mcts.cpp:152-169),
                  on 5x5, 9x9, 13x13 and 19x19 boards
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a, np.float32).tobytes()).hexdigest()


def main():
    if not O.ref_available():
        raise SystemExit("oracle/_ref/libazgo_ref.so is not built (make -C oracle with the reference present)")
    h = O._ref()
    import ctypes as C
    rng = {"next": {}, "uniform": {}, "normal": {}, "below7": {}, "derive": []}
    for seed in (0, 1, 42, 2 ** 63 + 5):
        out = (C.c_uint64 * 16)()
        h.ref_rng_next_u64(seed, 16, out)
        rng["next"][str(seed)] = [str(v) for v in out]
        for kind, key in ((1, "uniform"), (2, "normal"), (3, "below7")):
            d = (C.c_double * 16)()
            h.ref_rng_draws(seed, kind, 7, 16, d)
            rng[key][str(seed)] = [float(v).hex() for v in d]
    for args in ((1, 0xB4, 0, 0), (1, 3, 0, 0), (1, 3, 255, 0), (4, 3, 2, 1), (1, 2, 3, 4)):
        rng["derive"].append([list(args), str(h.ref_derive_seed(*args))])
    with open(os.path.join(HERE, "rng.json"), "w") as f:
        json.dump(rng, f, indent=1)

    weights = {}
    for tag, w in O.WORKLOADS.items():
        if tag == 4:
            continue   # the same network as workload 3
        ref = O.RefNetwork(w.cfg, 1)
        weights[str(tag)] = {name: sha(ref.get(name)) for name, _, _, _ in ref.layout()}
    with open(os.path.join(HERE, "weights.json"), "w") as f:
        json.dump(weights, f, indent=1)

    g = np.random.default_rng(2024)
    enc = {}
    for n in (5, 9, 19):
        stones = g.integers(0, 3, (3, n * n)).astype(np.uint8)   # three plies of history
        enc[f"stones_{n}"] = stones
        for to_move in (1, 2):
            for H in (1, 2, 8):
                for sym in range(8):
                    out = np.empty((2 * H + 2) * n * n, np.float32)
                    h.ref_encode_planes(stones.ctypes.data_as(C.POINTER(C.c_uint8)), 3, n, to_move, H, sym,
                                        O.fptr(out))
                    enc[f"planes_{n}_{to_move}_{H}_{sym}"] = out
    np.savez_compressed(os.path.join(HERE, "encode.npz"), **enc)

    w = O.WORKLOADS[1]
    net = O.init_network(w.cfg)
    ref = O.RefNetwork(w.cfg, 1)
    ref.load(net)
    inp, legal = O.workload_inputs(w, 8)
    logits, values = ref.infer(inp)
    np.savez_compressed(os.path.join(HERE, "infer_5x5_workload.npz"), input=inp, legal=legal, logits=logits,
                        values=values)

    cfg = O.make_cfg(9, 2, 16, value_hidden=16)
    net = O.random_network(cfg, 7)
    ref = O.RefNetwork(cfg, 7)
    ref.load(net)
    inp = np.random.default_rng(8).integers(0, 2, (4, cfg.planes, cfg.area)).astype(np.float32)
    logits, values = ref.infer(inp)
    tensors = {"t_" + k: v for k, v in net.tensors().items()}
    np.savez_compressed(os.path.join(HERE, "infer_9x9_random.npz"), input=inp, logits=logits, values=values,
                        **tensors)
    trunks()
    calibrated()
    games()
    print("golden vectors written to", HERE)


def reference_trunk(net, inp, blocks):
    """The reference's trunk after `blocks` blocks, [B][F][A], one channel
    per Network::infer through a policy head made an exact copy."""
    cfg = O.make_cfg(net.cfg.board, blocks, net.cfg.filters, net.cfg.value_hidden, net.cfg.history)
    ref = O.RefNetwork(cfg, 1)
    names = {name for name, _, _, _ in ref.layout()}
    for name, t in net.tensors().items():
        if name in names and not name.startswith("policy."):
            ref.set(name, t)
    F, A = cfg.filters, cfg.area
    ref.set("policy.bn.gamma", np.ones(2, np.float32))
    ref.set("policy.bn.beta", np.zeros(2, np.float32))
    ref.set("policy.bn.runMean", np.zeros(2, np.float32))
    ref.set("policy.bn.runVar", np.full(2, 1 - 1e-5, np.float32))
    assert np.float32(1) / np.sqrt(np.float32(1 - 1e-5) + np.float32(1e-5)) == 1
    fc = np.zeros((A + 1, 2 * A), np.float32)
    fc[np.arange(A), np.arange(A)] = 1
    ref.set("policy.fc.w", fc)
    ref.set("policy.fc.b", np.zeros(A + 1, np.float32))
    out = np.empty((inp.shape[0], F, A), np.float32)
    for c in range(F):
        w = np.zeros((2, F), np.float32)
        w[0, c] = 1
        ref.set("policy.conv.w", w)
        out[:, c] = ref.infer(inp)[0][:, :A]
    return out


def trunks():
    res = {}
    w = O.WORKLOADS[1]
    net = O.init_network(w.cfg)
    inp, _ = O.workload_inputs(w, 8)
    res["5x5/input"] = inp
    for k in (0, 2, 4):
        res[f"5x5/trunk{k}"] = reference_trunk(net, inp, k)
    cfg = O.make_cfg(9, 2, 16, value_hidden=16)
    net = O.random_network(cfg, 9)
    inp = np.random.default_rng(10).integers(0, 2, (3, cfg.planes, cfg.area)).astype(np.float32)
    res["9x9/input"] = inp
    res["9x9/trunk2"] = reference_trunk(net, inp, 2)
    np.savez_compressed(os.path.join(HERE, "trunk.npz"), **res)


# (board size, seeds, moves): lengths reach captures, ko fights (superko
# exclusions) and, on 19x19, superko lists longer than 512 positions.
GAMES = ((5, range(1, 11), 80), (9, range(1, 4), 200), (13, range(1, 2), 300), (19, range(1, 2), 600))


def games():
    out = {}
    for n, seeds, moves in GAMES:
        for seed in seeds:
            stones, to_move, hashes, legal = O.random_game(n, seed, moves, ref=True)
            key = f"{n}_{seed}"
            out[key + "/stones"], out[key + "/to_move"] = stones, to_move
            out[key + "/hashes"], out[key + "/legal"] = hashes, legal
    np.savez_compressed(os.path.join(HERE, "games.npz"), **out)


# Calibrated shapes: the workloads' networks (workload 4 is workload 3's)
# and the 19x19 preset's value head (configs/19x19.cfg: value_hidden 256).
CALIBRATED = {"1": O.WORKLOADS[1].cfg, "2": O.WORKLOADS[2].cfg, "3": O.WORKLOADS[3].cfg,
              "5": O.WORKLOADS[5].cfg, "3v256": O.make_cfg(19, 10, 128, value_hidden=256)}


def calibrated():
    seed = O.gen0_calibration_seed()
    out = {}
    for tag, cfg in CALIBRATED.items():
        ref = O.RefNetwork(cfg, 1)
        ref.calibrate_bn(seed, threads=os.cpu_count() or 1)
        for name, _, _, buf in ref.layout():
            if buf:
                out[f"{tag}/{name}"] = ref.get(name)
        print("calibrated", tag, flush=True)
    np.savez_compressed(os.path.join(HERE, "calibrated_bn.npz"), **out)

    w = O.WORKLOADS[1]
    inp, legal = O.workload_inputs(w, 8)
    res = {"input": inp, "legal": legal}
    for tag, cfg in (("4x32", w.cfg), ("2x16_own", O.make_cfg(5, 2, 16, ownership=1))):
        ref = O.RefNetwork(cfg, 1)
        ref.calibrate_bn(seed, threads=os.cpu_count() or 1)
        path = os.path.join(HERE, f"gen0_5x5_{tag}.azn")
        ref.save(path)
        back = O.RefNetwork.load_file(path, cfg)
        outs = back.infer(inp, ownership=bool(cfg.ownership))
        res[f"{tag}/logits"], res[f"{tag}/values"] = outs[0], outs[1]
        if cfg.ownership:
            res[f"{tag}/ownership"] = outs[2]
    np.savez_compressed(os.path.join(HERE, "gen0_infer.npz"), **res)


if __name__ == "__main__":
    if sys.argv[1:] == ["calibrated"]:
        calibrated()
    elif sys.argv[1:] == ["trunks"]:
        trunks()
    elif sys.argv[1:] == ["games"]:
        games()
    else:
        main()
