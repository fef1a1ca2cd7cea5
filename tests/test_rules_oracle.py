"""The oracle's restatement of the Go rules the legal moves need (Board::isLegal,
play, hashAfter, the Zobrist hash; Mcts::expand's superko filter), pinned by:

- the reference's own hand positions (tests/test_board.cpp:109-146,
  tests/test_game.cpp:19-65), restated;
- whole random games the reference's Game played (tests/golden/games.npz):
  the oracle plays the same games move for move, and every position's
  stones, side to move, hash and legal set match bit for bit;
- the invariant of tests/test_board.cpp:185-201: hashAfter(a) is the hash of
  the position play(a) reaches, for every legal a;
- where the reference's build is present (oracle/_ref), Board::isLegal and
  hashAfter themselves on every golden position, and on random boards no
  game reaches (groups without liberties, full boards).
"""
import os

import numpy as np
import pytest

import oracle as O
from _util import GOLDEN

B_, W_ = O.BLACK, O.WHITE


def rows(*lines):
    """boardFromRows (tests/): 'X' Black, 'O' White, '.' empty."""
    m = {".": 0, "X": B_, "O": W_}
    return np.array([m[ch] for line in lines for ch in line], np.uint8)


def pt(r, c, n=5):
    return r * n + c


def games():
    z = np.load(os.path.join(GOLDEN, "games.npz"))
    keys = sorted({k.split("/")[0] for k in z.files}, key=lambda k: tuple(map(int, k.split("_"))))
    for k in keys:
        n, seed = map(int, k.split("_"))
        yield n, seed, z[k + "/stones"], z[k + "/to_move"], z[k + "/hashes"], z[k + "/legal"]


def test_suicide_illegal():
    # tests/test_board.cpp:109-130
    eye = rows(".X...", "X....", ".....", ".....", ".....")
    lw = O.board_legal(eye, 5, W_)
    assert not lw[pt(0, 0)] and lw[25]
    assert O.board_legal(eye, 5, B_)[pt(0, 0)]
    multi = rows("O.X..", "XX...", ".....", ".....", ".....")
    assert not O.board_legal(multi, 5, W_)[pt(0, 1)]


def test_capture_that_looks_like_suicide_is_legal():
    # tests/test_board.cpp:132-146
    b = rows(".OX..", "OX...", "X....", ".....", ".....")
    assert O.board_legal(b, 5, B_)[pt(0, 0)]
    assert not O.board_legal(b, 5, W_)[pt(0, 0)]
    after, captured = O.play(b, 5, B_, pt(0, 0))
    assert captured == 2 and after[pt(0, 1)] == 0 and after[pt(1, 0)] == 0


def test_simple_ko_superko():
    # tests/test_game.cpp:19-55: Black takes at (2,2); the immediate retake
    # at (2,1) is a legal capture locally but recreates the start position.
    start = rows(".....", ".XO..", "XO.O.", ".XO..", ".....")
    take, retake = pt(2, 2), pt(2, 1)
    seen = [O.board_hash(start, 5)]
    assert O.legal_moves(start, 5, B_, seen)[take]
    after, cap = O.play(start, 5, B_, take)
    assert cap == 1 and after[retake] == 0
    seen.append(O.board_hash(after, 5))
    assert O.board_legal(after, 5, W_)[retake]                  # locally legal
    assert O.hash_after(after, 5, W_)[retake] == seen[0]          # recreates the start
    lg = O.legal_moves(after, 5, W_, seen)
    assert not lg[retake] and lg[25]
    # threat exchange elsewhere: the retake becomes legal
    b2, _ = O.play(after, 5, W_, pt(4, 4))
    seen.append(O.board_hash(b2, 5))
    b3, _ = O.play(b2, 5, B_, pt(0, 4))
    seen.append(O.board_hash(b3, 5))
    assert O.legal_moves(b3, 5, W_, seen)[retake]
    b4, cap = O.play(b3, 5, W_, retake)
    assert cap == 1 and b4[take] == 0
    seen.append(O.board_hash(b4, 5))
    assert O.board_legal(b4, 5, B_)[take] and not O.legal_moves(b4, 5, B_, seen)[take]


def test_pass_never_blocked():
    # tests/test_game.cpp:57-65: passing repeats a seen position, still legal
    empty = np.zeros(25, np.uint8)
    assert O.legal_moves(empty, 5, B_, [O.board_hash(empty, 5)])[25] == 1


def test_empty_board_hash_is_zero_and_keys_distinct():
    assert O.board_hash(np.zeros(81, np.uint8), 9) == 0
    keys = {O.zobrist_key(c, col) for c in range(441) for col in (B_, W_)}
    assert len(keys) == 882


def test_oracle_plays_the_golden_games():
    count = 0
    for n, seed, stones, to_move, hashes, legal in games():
        moves = len(stones) - 1
        got = O.random_game(n, seed, moves)
        for a, b in zip(got, (stones, to_move, hashes, legal)):
            assert np.array_equal(a, b), (n, seed)
        count += len(stones)
    assert count > 1500


def test_golden_positions_hash_and_legal():
    for n, seed, stones, to_move, hashes, legal in games():
        for i in range(0, len(stones), 7):
            assert O.board_hash(stones[i], n) == hashes[i]
            assert np.array_equal(O.legal_moves(stones[i], n, int(to_move[i]), hashes[:i + 1]), legal[i])


def test_hash_after_is_hash_of_play():
    for n, seed, stones, to_move, hashes, legal in games():
        for i in range(0, len(stones), 23):
            s, tm = stones[i], int(to_move[i])
            ha = O.hash_after(s, n, tm)
            bl = O.board_legal(s, n, tm)
            for a in np.flatnonzero(bl[:-1]):
                after, _ = O.play(s, n, tm, int(a))
                assert ha[a] == O.board_hash(after, n)
            assert ha[n * n] == hashes[i]


@pytest.mark.skipif(not O.ref_available(), reason="the reference's build (oracle/_ref) is not present")
def test_against_reference_board():
    import ctypes as C
    h = O._ref()
    for n, seed, stones, to_move, hashes, legal in games():
        for i in range(0, len(stones), 5):
            s = np.ascontiguousarray(stones[i])
            ref_legal = np.empty(n * n + 1, np.uint8)
            h.ref_board_legal(O.u8ptr(s), n, int(to_move[i]), O.u8ptr(ref_legal))
            assert np.array_equal(O.board_legal(s, n, int(to_move[i])), ref_legal)
            ref_ha = np.empty(n * n + 1, np.uint64)
            h.ref_hash_after(O.u8ptr(s), n, int(to_move[i]), ref_ha.ctypes.data_as(C.POINTER(C.c_uint64)))
            assert np.array_equal(O.hash_after(s, n, int(to_move[i])), ref_ha)
            assert h.ref_board_hash(O.u8ptr(s), n) == hashes[i]


def random_boards(n, count, seed):
    """Boards no game need reach (random stones: groups without liberties,
    full boards), both sides to move."""
    g = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        pe = g.uniform(0.02, 0.7)
        out.append(g.choice([0, 1, 2], size=n * n, p=[pe, (1 - pe) / 2, (1 - pe) / 2]).astype(np.uint8))
    return out


@pytest.mark.skipif(not O.ref_available(), reason="the reference's build (oracle/_ref) is not present")
def test_against_reference_on_random_boards():
    import ctypes as C
    h = O._ref()
    for n in (5, 9, 13, 19):
        for s in random_boards(n, 150, n):
            for tm in (B_, W_):
                rl = np.empty(n * n + 1, np.uint8)
                h.ref_board_legal(O.u8ptr(s), n, tm, O.u8ptr(rl))
                assert np.array_equal(O.board_legal(s, n, tm), rl)
                rh = np.empty(n * n + 1, np.uint64)
                h.ref_hash_after(O.u8ptr(s), n, tm, rh.ctypes.data_as(C.POINTER(C.c_uint64)))
                assert np.array_equal(O.hash_after(s, n, tm), rh)


def test_positions_workers_time_the_cpu_steps():
    """The CPU baseline of the steps either side of the pass (bench.py's
    positions leg): several threads encoding and finding legal moves with
    superko lists run for the budget and count what they did."""
    n = 9
    boards = random_boards(n, 12, 7)
    stones = np.stack(boards)
    to_move = np.array([B_, W_] * 6, np.uint8)
    g = np.random.default_rng(3)
    seen = [g.integers(0, 2 ** 63, k, dtype=np.int64).astype(np.uint64) for k in range(12)]
    one, el1 = O.time_positions_workers(stones, to_move, n, 8, seen, 1, 0.05)
    two, el2 = O.time_positions_workers(stones, to_move, n, 8, seen, 2, 0.05)
    assert el1 >= 0.05 and el2 >= 0.05
    assert one > 0 and two > 0
