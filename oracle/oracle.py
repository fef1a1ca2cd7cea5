"""The oracle's Python face (ctypes over liboracle.so and, when built, the
reference's own sources in _ref/libazgo_ref.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by the smoke check and by the
bench's CPU-baseline leg, to check results against. The product (the HIP library and its
binding under alphazero-go_amd/) never imports it.

The benchmark workloads (the five network/batch configurations the
measurements are quoted on) are defined here, with the synthetic-data
conventions the restatement in azgo_oracle.c documents.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libazgo_ref.so")


class Cfg(C.Structure):
    """NetConfig (include/azgo/network.hpp:24-36)."""
    _fields_ = [("board", C.c_int), ("history", C.c_int), ("blocks", C.c_int),
                ("filters", C.c_int), ("value_hidden", C.c_int), ("ownership", C.c_int)]

    @property
    def planes(self):
        return 2 * self.history + 2

    @property
    def area(self):
        return self.board * self.board

    @property
    def actions(self):
        return self.area + 1

    def key(self):
        return (self.board, self.history, self.blocks, self.filters, self.value_hidden, self.ownership)

    def __repr__(self):
        return (f"Cfg({self.board}x{self.board}, {self.blocks}x{self.filters}, V={self.value_hidden}"
                f"{', own' if self.ownership else ''})")


def make_cfg(board, blocks, filters, value_hidden=64, history=8, ownership=0):
    return Cfg(board, history, blocks, filters, value_hidden, ownership)


@dataclass
class Workload:
    """One benchmark workload: a network shape, a batch and its board distribution."""
    tag: int
    name: str
    cfg: Cfg
    batch: int
    p_black: float
    p_white: float
    batches: tuple = field(default_factory=tuple)

    def flops_per_position(self):
        """2 x multiply-adds of the convolutions and linear layers."""
        c = self.cfg
        A, P, F, V = c.area, c.planes, c.filters, c.value_hidden
        macs = F * 9 * P * A + 2 * c.blocks * F * 9 * F * A + 2 * F * A + 2 * A * (A + 1) + F * A + A * V + V
        return 2 * macs


WORKLOADS = {
    1: Workload(1, "5x5 4x32 b8", make_cfg(5, 4, 32), 8, 0.25, 0.25),
    2: Workload(2, "9x9 6x64 b64", make_cfg(9, 6, 64), 64, 0.25, 0.25),
    3: Workload(3, "19x19 10x128 b256", make_cfg(19, 10, 128), 256, 0.3, 0.3),
    4: Workload(4, "19x19 10x128 b1/8/32", make_cfg(19, 10, 128), 32, 0.3, 0.3, (1, 8, 32)),
    5: Workload(5, "19x19 20x256 b512", make_cfg(19, 20, 256), 512, 0.35, 0.35),
}

WEIGHT_SEED = 1


def _lib():
    if not hasattr(_lib, "h"):
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: {LIB_PATH} (run make -C oracle)")
        h = C.CDLL(LIB_PATH)
        P = C.POINTER
        f32, u8 = P(C.c_float), P(C.c_uint8)
        h.azo_splitmix64.argtypes = [P(C.c_uint64)]
        h.azo_splitmix64.restype = C.c_uint64
        h.azo_derive_seed.argtypes = [C.c_uint64] * 4
        h.azo_derive_seed.restype = C.c_uint64
        h.azo_rng_init.argtypes = [C.c_void_p, C.c_uint64]
        h.azo_rng_next.argtypes = [C.c_void_p]
        h.azo_rng_next.restype = C.c_uint64
        h.azo_rng_uniform.argtypes = [C.c_void_p]
        h.azo_rng_uniform.restype = C.c_double
        h.azo_rng_normal.argtypes = [C.c_void_p]
        h.azo_rng_normal.restype = C.c_double
        h.azo_rng_below.argtypes = [C.c_void_p, C.c_int]
        h.azo_rng_below.restype = C.c_int
        h.azo_tensor_count.argtypes = [P(Cfg)]
        h.azo_tensor_info.argtypes = [P(Cfg), C.c_int, C.c_char_p, C.c_size_t, P(C.c_size_t), P(C.c_size_t),
                                      P(C.c_int)]
        h.azo_arena_sizes.argtypes = [P(Cfg), P(C.c_size_t), P(C.c_size_t)]
        h.azo_init_network.argtypes = [P(Cfg), C.c_uint64, f32, f32]
        h.azo_synthetic_bn.argtypes = [P(Cfg), C.c_uint64, f32]
        h.azo_transform_point.argtypes = [C.c_int] * 3
        h.azo_encode_planes.argtypes = [u8, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, f32]
        h.azo_random_boards.argtypes = [C.c_int, C.c_int, C.c_uint64, C.c_uint64, C.c_double, C.c_double, u8, u8]
        h.azo_encode_batch.argtypes = [C.c_int, C.c_int, C.c_int, u8, u8, f32, u8]
        h.azo_blas_description.restype = C.c_char_p
        h.azo_im2col.argtypes = [f32, C.c_int, C.c_int, C.c_int, C.c_int, f32]
        h.azo_bn_infer.argtypes = [f32, f32, f32, f32, C.c_int, C.c_size_t, f32, f32]
        h.azo_conv3x3.argtypes = [C.c_int, f32, C.c_int, C.c_int, f32, C.c_int, C.c_int, f32, f32]
        h.azo_gemm.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, f32, f32, f32]
        h.azo_forward.argtypes = [P(Cfg), f32, f32, f32, C.c_int, C.c_int, f32, f32, f32]
        h.azo_trunk.argtypes = [P(Cfg), f32, f32, f32, C.c_int, C.c_int, C.c_int, f32]
        h.azo_forward_double.argtypes = [P(Cfg), f32, f32, f32, C.c_int, f32, f32, f32]
        h.azo_softmax_legal.argtypes = [f32, u8, C.c_int, C.c_int, f32]
        u64p = P(C.c_uint64)
        h.azo_zobrist_key.argtypes = [C.c_int, C.c_int]
        h.azo_zobrist_key.restype = C.c_uint64
        h.azo_legal_moves.argtypes = [u8, C.c_int, C.c_int, u64p, C.c_int, u8]
        h.azo_board_legal.argtypes = [u8, C.c_int, C.c_int, u8]
        h.azo_board_hash.argtypes = [u8, C.c_int]
        h.azo_board_hash.restype = C.c_uint64
        h.azo_hash_after.argtypes = [u8, C.c_int, C.c_int, u64p]
        h.azo_play.argtypes = [u8, C.c_int, C.c_int, C.c_int, u8]
        h.azo_random_game.argtypes = [C.c_int, C.c_uint64, C.c_int, u8, u8, u64p, u8]
        h.azo_time_workers.argtypes = [P(Cfg), f32, f32, f32, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                       P(C.c_double)]
        h.azo_time_workers.restype = C.c_double
        h.azo_time_positions_workers.argtypes = [C.c_int, C.c_int, C.c_int, u8, u8, u64p, P(C.c_int), C.c_int,
                                                 C.c_double, P(C.c_double)]
        h.azo_time_positions_workers.restype = C.c_double
        _lib.h = h
    return _lib.h


def fptr(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def u8ptr(a):
    return a.ctypes.data_as(C.POINTER(C.c_uint8))


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ------------------------------------------------------------------ rng

def splitmix64(x):
    s = C.c_uint64(x)
    v = _lib().azo_splitmix64(C.byref(s))
    return v, s.value


def derive_seed(a, b=0, c=0, d=0):
    return _lib().azo_derive_seed(a, b, c, d)


class Rng:
    def __init__(self, seed):
        self.state = (C.c_uint64 * 4)()
        _lib().azo_rng_init(self.state, seed)

    def next(self):
        return _lib().azo_rng_next(self.state)

    def uniform(self):
        return _lib().azo_rng_uniform(self.state)

    def normal(self):
        return _lib().azo_rng_normal(self.state)

    def below(self, n):
        return _lib().azo_rng_below(self.state, n)


# ------------------------------------------------------------------ network tensors

def layout(cfg):
    """[(name, size, offset, arena)] in params() then buffers() order."""
    h = _lib()
    out = []
    name = C.create_string_buffer(64)
    size, off, buf = C.c_size_t(), C.c_size_t(), C.c_int()
    for i in range(h.azo_tensor_count(C.byref(cfg))):
        h.azo_tensor_info(C.byref(cfg), i, name, 64, C.byref(size), C.byref(off), C.byref(buf))
        out.append((name.value.decode(), size.value, off.value, buf.value))
    return out


def arena_sizes(cfg):
    pf, bf = C.c_size_t(), C.c_size_t()
    _lib().azo_arena_sizes(C.byref(cfg), C.byref(pf), C.byref(bf))
    return pf.value, bf.value


class Net:
    """A network as the two ParamLayout arenas (params, buffers)."""

    def __init__(self, cfg, params, buffers):
        self.cfg, self.params, self.buffers = cfg, params, buffers

    def tensors(self):
        """{name: float32 view} in layout order."""
        d = {}
        for name, size, off, buf in layout(self.cfg):
            arena = self.buffers if buf else self.params
            d[name] = arena[off:off + size]
        return d


def init_network(cfg, seed=WEIGHT_SEED, synthetic_bn=True):
    """Network(cfg, seed) weights; synthetic BN statistics when asked."""
    pf, bf = arena_sizes(cfg)
    params = np.zeros(pf, np.float32)
    buffers = np.zeros(bf, np.float32)
    _lib().azo_init_network(C.byref(cfg), seed, fptr(params), fptr(buffers))
    if synthetic_bn:
        _lib().azo_synthetic_bn(C.byref(cfg), seed, fptr(buffers))
    return Net(cfg, params, buffers)


def random_network(cfg, seed, rng=None):
    """A network whose every tensor is random (for parity tests where the
    benchmark's BN convention would hide a wrong gamma/beta/bias): He weights
    from seed, then gamma ~ U(0.5, 1.5), beta/bias ~ U(-0.5, 0.5),
    mean ~ U(-1, 1), var ~ U(0.05, 2.05) from numpy's generator."""
    net = init_network(cfg, seed, synthetic_bn=False)
    g = np.random.default_rng(seed if rng is None else rng)
    for name, t in net.tensors().items():
        if name.endswith(".gamma"):
            t[:] = g.uniform(0.5, 1.5, t.size)
        elif name.endswith(".beta") or name.endswith(".b"):
            t[:] = g.uniform(-0.5, 0.5, t.size)
        elif name.endswith(".runMean"):
            t[:] = g.uniform(-1, 1, t.size)
        elif name.endswith(".runVar"):
            t[:] = g.uniform(0.05, 2.05, t.size)
    return net


# ------------------------------------------------------------------ boards

def transform_point(sym, p, n):
    return _lib().azo_transform_point(sym, p, n)


def encode_planes(stones, n, to_move, H, sym=0):
    """stones: uint8 [count][n*n] newest first; returns [2H+2][n*n]."""
    stones = np.ascontiguousarray(stones, np.uint8).reshape(-1, n * n)
    out = np.empty((2 * H + 2) * n * n, np.float32)
    _lib().azo_encode_planes(u8ptr(stones), stones.shape[0], n, to_move, H, sym, fptr(out))
    return out.reshape(2 * H + 2, n * n)


def random_boards(n, B, tag, p_black, p_white, seed=WEIGHT_SEED):
    stones = np.empty((B, n * n), np.uint8)
    to_move = np.empty(B, np.uint8)
    _lib().azo_random_boards(n, B, seed, tag, p_black, p_white, u8ptr(stones), u8ptr(to_move))
    return stones, to_move


def encode_batch(n, H, stones, to_move):
    B = stones.shape[0]
    inp = np.empty((B, 2 * H + 2, n * n), np.float32)
    legal = np.empty((B, n * n + 1), np.uint8)
    _lib().azo_encode_batch(n, H, B, u8ptr(np.ascontiguousarray(stones)), u8ptr(np.ascontiguousarray(to_move)),
                            fptr(inp), u8ptr(legal))
    return inp, legal


def workload_inputs(w: Workload, B=None, seed=WEIGHT_SEED):
    """(input [B][P][A], legal [B][A+1]) of a workload's synthetic positions."""
    B = w.batch if B is None else B
    stones, to_move = random_boards(w.cfg.board, B, w.tag, w.p_black, w.p_white, seed)
    return encode_batch(w.cfg.board, w.cfg.history, stones, to_move)


# ------------------------------------------------------------------ forward passes

NAIVE, BLAS = 0, 1


def blas_description():
    return _lib().azo_blas_description().decode()


def forward(net: Net, inp, mode=BLAS, ownership=False):
    cfg = net.cfg
    inp = _f32(inp)
    B = inp.shape[0]
    logits = np.empty((B, cfg.actions), np.float32)
    values = np.empty(B, np.float32)
    own = np.empty((B, cfg.area), np.float32) if ownership else None
    rc = _lib().azo_forward(C.byref(cfg), fptr(net.params), fptr(net.buffers), fptr(inp), B, mode,
                            fptr(logits), fptr(values), fptr(own) if own is not None else None)
    if rc == -2:
        raise RuntimeError("oracle: no CBLAS library could be loaded")
    if rc != 0:
        raise RuntimeError(f"oracle forward failed ({rc})")
    return (logits, values, own) if ownership else (logits, values)


def trunk(net: Net, inp, blocks=None, mode=BLAS):
    """The stem and the first `blocks` residual blocks (all by default) of
    the forward pass, [B][F][A]: the arithmetic of forward()."""
    cfg = net.cfg
    inp = _f32(inp)
    B = inp.shape[0]
    blocks = cfg.blocks if blocks is None else blocks
    out = np.empty((B, cfg.filters, cfg.area), np.float32)
    rc = _lib().azo_trunk(C.byref(cfg), fptr(net.params), fptr(net.buffers), fptr(inp), B, mode, blocks, fptr(out))
    if rc == -2:
        raise RuntimeError("oracle: no CBLAS library could be loaded")
    if rc != 0:
        raise RuntimeError(f"oracle trunk failed ({rc})")
    return out


def threaded(fn, inp, chunk, workers=None):
    """fn over inp in chunks of `chunk` positions on a pool of threads (the
    oracle's passes are single-threaded C calls that release the
    interpreter), concatenated in order: one position's outputs depend on
    its own input only."""
    from concurrent.futures import ThreadPoolExecutor
    workers = workers or max(1, min(16, len(os.sched_getaffinity(0))))
    parts = [inp[i:i + chunk] for i in range(0, len(inp), chunk)]
    with ThreadPoolExecutor(workers) as ex:
        outs = list(ex.map(fn, parts))
    if isinstance(outs[0], tuple):
        return tuple(np.concatenate([o[k] for o in outs]) for k in range(len(outs[0])))
    return np.concatenate(outs)


def forward_double(net: Net, inp, ownership=False):
    cfg = net.cfg
    inp = _f32(inp)
    B = inp.shape[0]
    logits = np.empty((B, cfg.actions), np.float32)
    values = np.empty(B, np.float32)
    own = np.empty((B, cfg.area), np.float32) if ownership else None
    rc = _lib().azo_forward_double(C.byref(cfg), fptr(net.params), fptr(net.buffers), fptr(inp), B,
                                   fptr(logits), fptr(values), fptr(own) if own is not None else None)
    if rc != 0:
        raise RuntimeError(f"oracle double forward failed ({rc})")
    return (logits, values, own) if ownership else (logits, values)


def im2col(x, C_, B, n, k):
    x = _f32(x)
    col = np.empty(C_ * k * k * B * n * n, np.float32)
    _lib().azo_im2col(fptr(x), C_, B, n, k, fptr(col))
    return col


def conv3x3(w, cin, cout, x, B, n, mode=NAIVE):
    """x [cin][B*n*n] channel-major -> [cout][B*n*n]."""
    x, w = _f32(x), _f32(w)
    col = np.empty(cin * 9 * B * n * n, np.float32)
    y = np.empty(cout * B * n * n, np.float32)
    rc = _lib().azo_conv3x3(mode, fptr(w), cin, cout, fptr(x), B, n, fptr(col), fptr(y))
    if rc:
        raise RuntimeError("oracle conv failed")
    return y


def bn_infer(gamma, beta, mean, var, x, C_, M):
    x = _f32(x)
    y = np.empty_like(x)
    _lib().azo_bn_infer(fptr(_f32(gamma)), fptr(_f32(beta)), fptr(_f32(mean)), fptr(_f32(var)), C_, M, fptr(x),
                        fptr(y))
    return y


def gemm(A, B, transB=False, mode=NAIVE):
    A, B = _f32(A), _f32(B)
    M, K = A.shape
    N = B.shape[0] if transB else B.shape[1]
    Cm = np.empty((M, N), np.float32)
    rc = _lib().azo_gemm(mode, int(transB), M, N, K, fptr(A), fptr(B), fptr(Cm))
    if rc:
        raise RuntimeError("oracle gemm failed")
    return Cm


def softmax_legal(logits, legal):
    logits = _f32(logits)
    legal = np.ascontiguousarray(legal, np.uint8)
    out = np.empty_like(logits)
    B, A1 = logits.shape
    _lib().azo_softmax_legal(fptr(logits), u8ptr(legal), B, A1, fptr(out))
    return out


# ------------------------------------------------------------------ rules (legal moves, superko)

EMPTY, BLACK, WHITE = 0, 1, 2


def _u64p(a):
    return a.ctypes.data_as(C.POINTER(C.c_uint64))


def zobrist_key(padded_cell, color):
    return _lib().azo_zobrist_key(padded_cell, color)


def board_hash(stones, n):
    s = np.ascontiguousarray(stones, np.uint8)
    return _lib().azo_board_hash(u8ptr(s), n)


def legal_moves(stones, n, to_move, seen=()):
    """Mcts::expand's legal set: Board::isLegal and no superko repeat of `seen`."""
    s = np.ascontiguousarray(stones, np.uint8)
    h = np.ascontiguousarray(np.asarray(seen, np.uint64).reshape(-1))
    out = np.empty(n * n + 1, np.uint8)
    _lib().azo_legal_moves(u8ptr(s), n, to_move, _u64p(h), h.size, u8ptr(out))
    return out


def board_legal(stones, n, to_move):
    s = np.ascontiguousarray(stones, np.uint8)
    out = np.empty(n * n + 1, np.uint8)
    _lib().azo_board_legal(u8ptr(s), n, to_move, u8ptr(out))
    return out


def hash_after(stones, n, to_move):
    s = np.ascontiguousarray(stones, np.uint8)
    out = np.empty(n * n + 1, np.uint64)
    _lib().azo_hash_after(u8ptr(s), n, to_move, _u64p(out))
    return out


def play(stones, n, to_move, action):
    """(stones after the move, stones captured)."""
    s = np.ascontiguousarray(stones, np.uint8)
    out = np.empty(n * n, np.uint8)
    captured = _lib().azo_play(u8ptr(s), n, to_move, action, u8ptr(out))
    return out, captured


def random_game(n, seed, moves, ref=False):
    """Every position of a random game (bnCalibrationPositions' move choice):
    (stones [k+1][n*n], to_move [k+1], hashes [k+1], legal [k+1][n*n+1]).
    ref=True plays it with the reference's own Game (oracle/_ref)."""
    area = n * n
    stones = np.zeros((moves + 1, area), np.uint8)
    to_move = np.zeros(moves + 1, np.uint8)
    hashes = np.zeros(moves + 1, np.uint64)
    legal = np.zeros((moves + 1, area + 1), np.uint8)
    fn = _ref().ref_random_game if ref else _lib().azo_random_game
    k = fn(n, seed, moves, u8ptr(stones), u8ptr(to_move), _u64p(hashes), u8ptr(legal))
    return stones[:k + 1], to_move[:k + 1], hashes[:k + 1], legal[:k + 1]


def time_workers(net: Net, inp, workers, calls, mode=BLAS, warm=True):
    """Positions/s of `workers` threads each running `calls` single-threaded
    passes over inp (after one warm-up pass when `warm`); returns (rate,
    elapsed seconds)."""
    inp = _f32(inp)
    el = C.c_double()
    rate = _lib().azo_time_workers(C.byref(net.cfg), fptr(net.params), fptr(net.buffers), fptr(inp), inp.shape[0],
                                   mode, workers, calls, int(warm), C.byref(el))
    return rate, el.value


def time_positions_workers(stones, to_move, n, H, seen, workers, budget):
    """Positions/s of `workers` threads each encoding and finding the legal
    moves (superko list seen[b] for position b) of the positions in turn for
    `budget` seconds; returns (rate, elapsed seconds)."""
    st = np.ascontiguousarray(stones, np.uint8).reshape(-1, n * n)
    tm = np.ascontiguousarray(to_move, np.uint8)
    lists = [np.asarray(x, np.uint64).reshape(-1) for x in seen]
    offsets = np.zeros(len(lists) + 1, np.int32)
    offsets[1:] = np.cumsum([x.size for x in lists])
    flat = np.ascontiguousarray(np.concatenate(lists) if lists else np.zeros(0, np.uint64))
    el = C.c_double()
    rate = _lib().azo_time_positions_workers(n, H, st.shape[0], u8ptr(st), u8ptr(tm), _u64p(flat),
                                             offsets.ctypes.data_as(C.POINTER(C.c_int)), workers, budget,
                                             C.byref(el))
    return rate, el.value


# ------------------------------------------------------------------ metrics

def max_err(x, ref):
    """maxErr = max|x - ref| / max|ref| (tests/test_cuda.cpp:150-171)."""
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.abs(ref).max()
    num = np.abs(x - ref).max()
    return num / den if den > 0 else num


def legal_argmax(logits, legal):
    """Argmax over legal actions, ties to the lowest index."""
    masked = np.where(np.asarray(legal, bool), logits, -np.inf)
    return masked.argmax(axis=1)


# ------------------------------------------------------------------ the reference compiled from source

def ref_available():
    return os.path.exists(REF_PATH)


def _ref():
    if not hasattr(_ref, "h"):
        h = C.CDLL(REF_PATH)
        P = C.POINTER
        f32, u8 = P(C.c_float), P(C.c_uint8)
        h.ref_splitmix64.argtypes = [P(C.c_uint64)]
        h.ref_splitmix64.restype = C.c_uint64
        h.ref_derive_seed.argtypes = [C.c_uint64] * 4
        h.ref_derive_seed.restype = C.c_uint64
        h.ref_rng_draws.argtypes = [C.c_uint64, C.c_int, C.c_int, C.c_int, P(C.c_double)]
        h.ref_rng_next_u64.argtypes = [C.c_uint64, C.c_int, P(C.c_uint64)]
        h.ref_transform_point.argtypes = [C.c_int] * 3
        h.ref_encode_planes.argtypes = [u8, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, f32]
        h.ref_network_new.argtypes = [C.c_int] * 6 + [C.c_uint64]
        h.ref_network_new.restype = C.c_void_p
        h.ref_network_free.argtypes = [C.c_void_p]
        h.ref_layout_count.argtypes = [C.c_void_p]
        h.ref_layout_entry.argtypes = [C.c_void_p, C.c_int, C.c_char_p, C.c_size_t, P(C.c_size_t), P(C.c_size_t),
                                       P(C.c_int)]
        h.ref_layout_sizes.argtypes = [C.c_void_p, P(C.c_size_t), P(C.c_size_t)]
        h.ref_tensor_get.argtypes = [C.c_void_p, C.c_char_p, f32]
        h.ref_tensor_get.restype = C.c_long
        h.ref_tensor_set.argtypes = [C.c_void_p, C.c_char_p, f32]
        h.ref_tensor_set.restype = C.c_long
        h.ref_network_infer.argtypes = [C.c_void_p, f32, C.c_int, f32, f32, f32]
        h.ref_im2col.argtypes = [f32, C.c_int, C.c_int, C.c_int, C.c_int, f32]
        h.ref_conv_forward.argtypes = [f32, C.c_int, C.c_int, C.c_int, f32, C.c_int, C.c_int, f32]
        h.ref_bn_infer.argtypes = [f32, f32, f32, f32, C.c_int, C.c_int, f32, f32]
        h.ref_calibrate_bn.argtypes = [C.c_void_p, C.c_uint64, C.c_int]
        h.ref_bn_calibration_positions.argtypes = [C.c_int, C.c_int, C.c_uint64, C.c_int, f32]
        h.ref_save_network.argtypes = [C.c_void_p, C.c_char_p, C.c_char_p, C.c_size_t]
        h.ref_load_network.argtypes = [C.c_char_p, C.c_char_p, C.c_size_t]
        h.ref_load_network.restype = C.c_void_p
        u64p = P(C.c_uint64)
        h.ref_random_game.argtypes = [C.c_int, C.c_uint64, C.c_int, u8, u8, u64p, u8]
        h.ref_board_legal.argtypes = [u8, C.c_int, C.c_int, u8]
        h.ref_hash_after.argtypes = [u8, C.c_int, C.c_int, u64p]
        h.ref_board_hash.argtypes = [u8, C.c_int]
        h.ref_board_hash.restype = C.c_uint64
        _ref.h = h
    return _ref.h


# The seed generation 0's batch-norm calibration uses: deriveSeed(seed = 1,
# 0, kPhaseBatchNorm = 7) (src/trainer.cpp:559; include/azgo/run_state.hpp:120;
# the config's default seed, include/azgo/config.hpp:39).
PHASE_BATCH_NORM = 7


def gen0_calibration_seed(seed=WEIGHT_SEED):
    return derive_seed(seed, 0, PHASE_BATCH_NORM)


class RefNetwork:
    """azgo::Network built by the reference's own code."""

    def __init__(self, cfg, seed, _ptr=None):
        self.cfg = cfg
        self.h = _ref()
        self.ptr = _ptr if _ptr is not None else self.h.ref_network_new(
            cfg.board, cfg.history, cfg.blocks, cfg.filters, cfg.value_hidden, cfg.ownership, seed)

    @classmethod
    def load_file(cls, path, cfg):
        """loadNetwork(path) (src/checkpoint.cpp:102-124); raises with its message."""
        err = C.create_string_buffer(512)
        ptr = _ref().ref_load_network(os.fsencode(path), err, 512)
        if not ptr:
            raise RuntimeError(err.value.decode())
        return cls(cfg, 0, _ptr=ptr)

    def save(self, path):
        """saveNetwork (src/checkpoint.cpp:84-100)."""
        err = C.create_string_buffer(512)
        if self.h.ref_save_network(self.ptr, os.fsencode(path), err, 512):
            raise RuntimeError(err.value.decode())

    def calibrate_bn(self, seed, threads=8):
        """calibrateBatchNorm (src/bn_calibration.cpp:33-45)."""
        self.h.ref_calibrate_bn(self.ptr, seed, threads)

    def __del__(self):
        if getattr(self, "ptr", None):
            self.h.ref_network_free(self.ptr)
            self.ptr = None

    def layout(self):
        out = []
        name = C.create_string_buffer(64)
        size, off, buf = C.c_size_t(), C.c_size_t(), C.c_int()
        for i in range(self.h.ref_layout_count(self.ptr)):
            self.h.ref_layout_entry(self.ptr, i, name, 64, C.byref(size), C.byref(off), C.byref(buf))
            out.append((name.value.decode(), size.value, off.value, buf.value))
        return out

    def sizes(self):
        pf, bf = C.c_size_t(), C.c_size_t()
        self.h.ref_layout_sizes(self.ptr, C.byref(pf), C.byref(bf))
        return pf.value, bf.value

    def get(self, name):
        n = self.h.ref_tensor_get(self.ptr, name.encode(), None)
        out = np.empty(n, np.float32)
        self.h.ref_tensor_get(self.ptr, name.encode(), fptr(out))
        return out

    def set(self, name, values):
        v = _f32(values)
        if self.h.ref_tensor_set(self.ptr, name.encode(), fptr(v)) != v.size:
            raise KeyError(name)

    def load(self, net: Net):
        for name, t in net.tensors().items():
            self.set(name, t)

    def infer(self, inp, ownership=False):
        inp = _f32(inp)
        B = inp.shape[0]
        logits = np.empty((B, self.cfg.actions), np.float32)
        values = np.empty(B, np.float32)
        own = np.empty((B, self.cfg.area), np.float32) if ownership else None
        self.h.ref_network_infer(self.ptr, fptr(inp), B, fptr(logits), fptr(values),
                                 fptr(own) if own is not None else None)
        return (logits, values, own) if ownership else (logits, values)
