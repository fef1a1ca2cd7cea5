"""The steps either side of the pass on the GPU, through the C ABI, against
the oracle (byte and integer work: bit for bit):

- azh_encode_planes: encodePlanes (src/encode.cpp:14-43) for every board
  size, history length, number of plies present, side to move and symmetry,
  against the oracle and against planes the reference itself encoded
  (tests/golden/encode.npz);
- azh_legal_moves: Mcts::expand's legal set (Board::isLegal + positional
  superko, src/mcts.cpp:152-169) on every position of the reference's random
  games (tests/golden/games.npz; superko lists up to 601 hashes), on the
  reference's hand positions (suicide, capture, ko), and on random boards no
  game reaches, with superko lists that forbid some of the legal moves;
- azh_evaluate_positions: the whole leaf evaluation (encode, pass, legal
  moves, logits mapped back from the symmetry, priors) on game positions with
  history and random symmetries, against the oracle's encode + blas pass +
  legal moves + softmax on a calibrated generation-0 network (max-abs 1e-4 on
  logits and values).
"""
import os

import numpy as np
import pytest

import oracle as O
from _util import GOLDEN, calibrated_network, to_hip_cfg
from test_rules_oracle import games, random_boards, rows, pt

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [5, 9, 13, 19])
def test_encode_vs_oracle(hip, n):
    g = np.random.default_rng(n)
    A = n * n
    for H in (1, 2, 8):
        B = 24
        stones = g.integers(0, 3, (B, H, A)).astype(np.uint8)
        plies = g.integers(1, H + 1, B).astype(np.int32)
        to_move = g.integers(1, 3, B).astype(np.uint8)
        sym = g.integers(0, 8, B).astype(np.uint8)
        got = hip.encode_planes(stones, to_move, n, H, plies, sym)
        for b in range(B):
            want = O.encode_planes(stones[b, :plies[b]], n, int(to_move[b]), H, int(sym[b]))
            assert np.array_equal(got[b].view(np.uint32), want.view(np.uint32)), (n, H, b)
        # all plies present, identity symmetry
        got = hip.encode_planes(stones, to_move, n, H)
        for b in range(B):
            assert np.array_equal(got[b], O.encode_planes(stones[b], n, int(to_move[b]), H, 0))


def test_encode_vs_reference_planes(hip):
    z = np.load(os.path.join(GOLDEN, "encode.npz"))
    for n in (5, 9, 19):
        stones = z[f"stones_{n}"]   # three plies
        for to_move in (1, 2):
            for H in (1, 2, 8):
                padded = np.zeros((8, H, n * n), np.uint8)
                padded[:, :min(3, H)] = stones[:min(3, H)]
                got = hip.encode_planes(padded, np.full(8, to_move, np.uint8), n, H,
                                        np.full(8, min(3, H), np.int32), np.arange(8, dtype=np.uint8))
                for sym in range(8):
                    want = z[f"planes_{n}_{to_move}_{H}_{sym}"].reshape(2 * H + 2, n * n)
                    assert np.array_equal(got[sym], want), (n, to_move, H, sym)


def test_legal_moves_on_reference_games(hip):
    total = 0
    for n, seed, stones, to_move, hashes, legal in games():
        seen = [hashes[:i + 1] for i in range(len(stones))]
        got = hip.legal_moves(stones, to_move, n, seen)
        assert np.array_equal(got, legal), (n, seed, np.argwhere(got != legal)[:5])
        total += len(stones)
    print(f"{total} positions")


def test_legal_moves_hand_positions(hip):
    # tests/test_board.cpp:109-146 and tests/test_game.cpp:19-55, restated
    eye = rows(".X...", "X....", ".....", ".....", ".....")
    multi = rows("O.X..", "XX...", ".....", ".....", ".....")
    cap = rows(".OX..", "OX...", "X....", ".....", ".....")
    start = rows(".....", ".XO..", "XO.O.", ".XO..", ".....")
    after, _ = O.play(start, 5, 1, pt(2, 2))
    boards = np.stack([eye, eye, multi, cap, cap, after])
    to_move = np.array([2, 1, 2, 1, 2, 2], np.uint8)
    seen = [[], [], [], [], [], [O.board_hash(start, 5), O.board_hash(after, 5)]]
    got = hip.legal_moves(boards, to_move, 5, seen)
    assert not got[0, pt(0, 0)] and got[1, pt(0, 0)]
    assert not got[2, pt(0, 1)]
    assert got[3, pt(0, 0)] and not got[4, pt(0, 0)]
    assert not got[5, pt(2, 1)] and got[5, 25]   # the ko retake, forbidden by superko
    for b in range(len(boards)):
        assert np.array_equal(got[b], O.legal_moves(boards[b], 5, int(to_move[b]), seen[b]))


@pytest.mark.parametrize("n", [5, 9, 13, 19])
def test_legal_moves_random_boards(hip, n):
    """Boards no game reaches (groups without liberties, full boards, lone
    empty points), both sides to move; each superko list holds some of the
    position's own hashes after a legal move (so those moves become illegal)
    and random hashes, up to 1100 entries (several LDS chunks)."""
    g = np.random.default_rng(100 + n)
    boards = random_boards(n, 40, 200 + n)
    boards += [np.full(n * n, 1, np.uint8), np.full(n * n, 2, np.uint8)]
    one = np.full(n * n, 2, np.uint8)
    one[n * n // 2] = 0
    boards.append(one)
    stones, to_move, seen = [], [], []
    for s in boards:
        for tm in (1, 2):
            ha = O.hash_after(s, n, tm)
            lg = O.board_legal(s, n, tm)
            cand = ha[:-1][lg[:-1] == 1]
            pick = cand[g.random(cand.size) < 0.3]
            junk = g.integers(0, 2 ** 63, int(g.integers(0, 1100)), dtype=np.int64).astype(np.uint64)
            lst = np.concatenate([pick, junk])
            g.shuffle(lst)
            stones.append(s)
            to_move.append(tm)
            seen.append(lst)
    stones = np.stack(stones)
    to_move = np.array(to_move, np.uint8)
    got = hip.legal_moves(stones, to_move, n, seen)
    for b in range(len(stones)):
        want = O.legal_moves(stones[b], n, int(to_move[b]), seen[b])
        assert np.array_equal(got[b], want), (n, b, np.flatnonzero(got[b] != want))


def test_legal_moves_argument_checks(hip):
    s = np.zeros((1, 25), np.uint8)
    with pytest.raises(hip.HipError):
        hip.legal_moves(s, np.array([3], np.uint8), 5)      # no side to move
    bad = s.copy()
    bad[0, 3] = 7
    with pytest.raises(hip.HipError):
        hip.legal_moves(bad, np.array([1], np.uint8), 5)    # not a stone byte


def _history(stones, i, H):
    """Mcts::evaluateLeaves' history at a root (src/mcts.cpp:119-132): the
    position i, then the game's earlier ones, newest first, at most H."""
    k = min(H, i + 1)
    hist = np.zeros((H, stones.shape[1]), np.uint8)
    hist[:k] = stones[i::-1][:k]
    return hist, k


@pytest.mark.parametrize("n,tag", [(5, "1"), (9, "2"), (19, "3")])
def test_evaluate_positions_end_to_end(hip, n, tag):
    net = calibrated_network(tag)
    H = net.cfg.history
    g = np.random.default_rng(7 + n)
    pos = [(n_, s, st, tm, hs, lg) for (n_, s, st, tm, hs, lg) in games() if n_ == n]
    B = 32 if n < 19 else 16
    hist, plies, to_move, sym, seen, legal_ref, idx = [], [], [], [], [], [], []
    for b in range(B):
        _, _, st, tm, hs, lg = pos[b % len(pos)]
        i = int(g.integers(0, len(st)))
        h, k = _history(st, i, H)
        hist.append(h)
        plies.append(k)
        to_move.append(tm[i])
        sym.append(g.integers(0, 8))
        seen.append(hs[:i + 1])
        legal_ref.append(lg[i])
    hist = np.stack(hist)
    plies = np.array(plies, np.int32)
    to_move = np.array(to_move, np.uint8)
    sym = np.array(sym, np.uint8)
    with hip.Runner(to_hip_cfg(hip, net.cfg), net.tensors(), B, 1) as r:
        logits, priors, legal, values = r.evaluate_positions(hist, to_move, plies, sym, seen)
    assert np.array_equal(legal, np.stack(legal_ref))
    # The oracle: encode with the symmetry, the blas pass, logits mapped back.
    planes = np.stack([O.encode_planes(hist[b, :plies[b]], n, int(to_move[b]), H, int(sym[b])) for b in range(B)])
    ref_logits, ref_values = O.forward(net, planes, O.BLAS)
    A = n * n
    mapped = np.empty_like(ref_logits)
    for b in range(B):
        t = [O.transform_point(int(sym[b]), a, n) for a in range(A)] + [A]
        mapped[b] = ref_logits[b][t]
    dl = float(np.abs(logits.astype(np.float64) - mapped).max())
    dv = float(np.abs(values.astype(np.float64) - ref_values).max())
    ref_priors = O.softmax_legal(mapped, legal)
    dp = float(np.abs(priors.astype(np.float64) - ref_priors).max())
    print(f"{n}x{n} B={B}: logits {dl:.3g} values {dv:.3g} priors {dp:.3g}")
    assert dl <= 1e-4 and dv <= 1e-4
    assert dp <= 1e-5
    assert np.all(priors[legal == 0] == 0)
    assert np.allclose(priors.sum(axis=1), 1.0, atol=1e-5)


def test_time_positions_runs_each_step(hip):
    net = calibrated_network("1")
    n, H = 5, net.cfg.history
    g = np.random.default_rng(3)
    B = 8
    stones = g.integers(0, 3, (B, H, n * n)).astype(np.uint8)
    to_move = g.integers(1, 3, B).astype(np.uint8)
    with hip.Runner(to_hip_cfg(hip, net.cfg), net.tensors(), B, 1) as r:
        ms = r.time_positions(stones, to_move, iters=3)
        assert all(x > 0 for x in ms) and ms[3] >= max(ms[:3])
        # the slot is idle again: an evaluation after the timing works
        logits, priors, legal, values = r.evaluate_positions(stones, to_move)
    assert np.isfinite(logits).all() and np.isfinite(values).all()


def _game_positions(n, H, B, seed):
    """B game positions of board n with history, random symmetries and their
    superko lists (as test_evaluate_positions_end_to_end draws them)."""
    g = np.random.default_rng(seed)
    pos = [(n_, s, st, tm, hs, lg) for (n_, s, st, tm, hs, lg) in games() if n_ == n]
    hist, plies, to_move, sym, seen = [], [], [], [], []
    for b in range(B):
        _, _, st, tm, hs, lg = pos[b % len(pos)]
        i = int(g.integers(0, len(st)))
        h, k = _history(st, i, H)
        hist.append(h)
        plies.append(k)
        to_move.append(tm[i])
        sym.append(g.integers(0, 8))
        seen.append(hs[:i + 1])
    return (np.stack(hist), np.array(to_move, np.uint8), np.array(plies, np.int32), np.array(sym, np.uint8), seen)


@pytest.mark.parametrize("n,tag", [(9, "2"), (19, "3")])
def test_begin_positions_equals_evaluate(hip, n, tag):
    """azh_begin_positions (asynchronous, per-slot pinned stone staging)
    gives azh_evaluate_positions' outputs bit for bit: two slots in flight at
    once on different batches, then a smaller batch on a slot that held a
    larger one (the outputs' packing follows the batch size)."""
    import threading
    net = calibrated_network(tag)
    H = net.cfg.history
    B = 24 if n < 19 else 16
    first = _game_positions(n, H, B, 40 + n)
    second = _game_positions(n, H, B, 50 + n)
    small = tuple(a[:5] if isinstance(a, np.ndarray) else a[:5] for a in second)
    with hip.Runner(to_hip_cfg(hip, net.cfg), net.tensors(), B, 2) as r:
        want = [r.evaluate_positions(*first), r.evaluate_positions(*second), r.evaluate_positions(*small)]
        events = [threading.Event(), threading.Event()]
        errors = []

        def done(slot, err):
            if err:
                errors.append(err)
            events[slot].set()

        r.begin_positions(0, done, *first)
        r.begin_positions(1, done, *second)
        for e in events:
            assert e.wait(60)
        assert not errors, errors
        got = [r.position_outputs(0, B), r.position_outputs(1, B)]
        events[0].clear()
        r.begin_positions(0, done, *small)
        assert events[0].wait(60) and not errors
        got.append(r.position_outputs(0, 5))
    for g_, w_ in zip(got, want):
        # logits mapped back, priors, legal, values
        for a, b in zip(g_, (w_[0], w_[1], w_[2], w_[3])):
            assert a.shape == b.shape and a.tobytes() == b.tobytes()


def test_begin_positions_refusals(hip):
    """Bad positions fail the call before the slot is claimed (the slot
    stays usable), as does a busy slot; the pass after them is right."""
    import threading
    net = calibrated_network("1")
    n, H, B = 5, net.cfg.history, 6
    stones, to_move, plies, sym, seen = _game_positions(n, H, B, 77)
    with hip.Runner(to_hip_cfg(hip, net.cfg), net.tensors(), B, 1) as r:
        want = r.evaluate_positions(stones, to_move, plies, sym, seen)
        ev = threading.Event()
        bad = stones.copy()
        bad[0, 0, 0] = 3
        with pytest.raises(hip.HipError, match="stone byte"):
            r.begin_positions(0, lambda s, e: ev.set(), bad, to_move, plies, sym, seen)
        bad_turn = to_move.copy()
        bad_turn[1] = 0
        with pytest.raises(hip.HipError, match="side to move"):
            r.begin_positions(0, lambda s, e: ev.set(), stones, bad_turn, plies, sym, seen)
        hip.set_copy_out_delay(200000)   # the pass holds the slot for 0.2 s
        try:
            r.begin_positions(0, lambda s, e: ev.set(), stones, to_move, plies, sym, seen)
            with pytest.raises(hip.HipError, match="in flight"):
                r.begin_positions(0, lambda s, e: None, stones, to_move, plies, sym, seen)
            assert ev.wait(60)
        finally:
            hip.set_copy_out_delay(0)
        got = r.position_outputs(0, B)
    for a, b in zip(got, want):
        assert a.tobytes() == b.tobytes()


def test_positions_kept_full_and_failure(hip):
    """azh_time_pipelined_positions keeps both slots busy through
    azh_begin_positions: every pass completes once and both slots hold the
    synchronous outputs afterwards; an injected failure (the runner's
    fail-after-n hook) comes back through done, stops the resubmission and
    leaves both slots usable."""
    net = calibrated_network("2")
    n, H, B = 9, net.cfg.history, 20
    stones, to_move, plies, sym, seen = _game_positions(n, H, B, 91)
    with hip.Runner(to_hip_cfg(hip, net.cfg), net.tensors(), B, 2) as r:
        want = r.evaluate_positions(stones, to_move, plies, sym, seen)
        before = hip.passes_completed()
        ms = r.time_pipelined_positions(B, 7, stones, to_move, plies, sym, seen)
        assert ms > 0 and hip.passes_completed() - before == 7
        for slot in (0, 1):
            for a, b in zip(r.position_outputs(slot, B), want):
                assert a.tobytes() == b.tobytes()
        hip.fail_passes_after(2)
        try:
            with pytest.raises(hip.HipError, match="injected failure"):
                r.time_pipelined_positions(B, 12, stones, to_move, plies, sym, seen)
        finally:
            hip.fail_passes_after(0)
        assert r.time_pipelined_positions(B, 2, stones, to_move, plies, sym, seen) > 0
        for a, b in zip(r.position_outputs(0, B), want):
            assert a.tobytes() == b.tobytes()


def test_begin_positions_defaults(hip):
    """No plies (all H present), no symmetry and no superko lists, one
    position and a full batch: the asynchronous pass equals the synchronous
    one bit for bit."""
    import threading
    net = calibrated_network("1")
    n, H = 5, net.cfg.history
    g = np.random.default_rng(12)
    with hip.Runner(to_hip_cfg(hip, net.cfg), net.tensors(), 16, 1) as r:
        for B in (1, 16):
            stones = g.integers(0, 3, (B, H, n * n)).astype(np.uint8)
            to_move = g.integers(1, 3, B).astype(np.uint8)
            want = r.evaluate_positions(stones, to_move)
            ev = threading.Event()
            r.begin_positions(0, lambda s, e: ev.set(), stones, to_move)
            assert ev.wait(60)
            for a, b in zip(r.position_outputs(0, B), want):
                assert a.tobytes() == b.tobytes()
