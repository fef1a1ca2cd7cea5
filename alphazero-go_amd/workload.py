"""The benchmark workloads (five network/batch configurations) and their
seeded data, from workload/azgo_workload.cpp (libazgo_workload.so): the
tensors of Network(cfg, seed) with the workloads' synthetic BN statistics,
and synthetic encoded positions with their legal-move masks.

cfg tuples are (board, history, blocks, filters, value_hidden).
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libazgo_workload.so")
SEED = 1


@dataclass
class Workload:
    tag: int
    name: str
    cfg: tuple
    batch: int
    p_black: float
    p_white: float
    batches: tuple = field(default_factory=tuple)

    @property
    def board(self):
        return self.cfg[0]

    def flops_per_position(self):
        """2 x multiply-adds of the convolutions and linear layers."""
        n, H, blocks, F, V = self.cfg
        A, P = n * n, 2 * H + 2
        macs = F * 9 * P * A + 2 * blocks * F * 9 * F * A + 2 * F * A + 2 * A * (A + 1) + F * A + A * V + V
        return 2 * macs

    def stem_conv_flops(self, B):
        """The stem convolution (2H + 2 input planes to F channels) over B positions."""
        n, H, blocks, F, V = self.cfg
        return 2.0 * F * 9 * (2 * H + 2) * n * n * B

    def trunk_conv_flops(self, B):
        """One residual-tower convolution over B positions."""
        n, H, blocks, F, V = self.cfg
        return 2.0 * F * 9 * F * n * n * B


WORKLOADS = {
    1: Workload(1, "5x5 4x32 batch 8", (5, 8, 4, 32, 64), 8, 0.25, 0.25),
    2: Workload(2, "9x9 6x64 batch 64", (9, 8, 6, 64, 64), 64, 0.25, 0.25),
    3: Workload(3, "19x19 10x128 batch 256", (19, 8, 10, 128, 64), 256, 0.3, 0.3),
    4: Workload(4, "19x19 10x128 batch 1/8/32", (19, 8, 10, 128, 64), 32, 0.3, 0.3, (1, 8, 32)),
    5: Workload(5, "19x19 20x256 batch 512", (19, 8, 20, 256, 64), 512, 0.35, 0.35),
}


def _lib():
    if not hasattr(_lib, "h"):
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"workload generator not built: {LIB_PATH}")
        h = C.CDLL(LIB_PATH)
        i = C.c_int
        h.azw_tensor_count.argtypes = [i] * 5
        h.azw_tensor_info.argtypes = [i] * 6 + [C.c_char_p, C.c_size_t, C.POINTER(C.c_size_t)]
        h.azw_network.argtypes = [i] * 5 + [C.c_uint64, C.POINTER(C.c_float)]
        h.azw_positions.argtypes = [i, i, i, C.c_uint64, C.c_uint64, C.c_double, C.c_double,
                                    C.POINTER(C.c_float), C.POINTER(C.c_uint8)]
        h.azw_stones.argtypes = [i, i, C.c_uint64, C.c_uint64, C.c_double, C.c_double, C.POINTER(C.c_uint8),
                                 C.POINTER(C.c_uint8)]
        _lib.h = h
    return _lib.h


def tensor_list(cfg):
    """[(name, size)] in params() then buffers() order."""
    h = _lib()
    name = C.create_string_buffer(64)
    size = C.c_size_t()
    out = []
    for i in range(h.azw_tensor_count(*cfg)):
        h.azw_tensor_info(*cfg, i, name, 64, C.byref(size))
        out.append((name.value.decode(), size.value))
    return out


def network_tensors(cfg, seed=SEED):
    """{name: float32 array} of the seeded network with synthetic BN stats."""
    lst = tensor_list(cfg)
    flat = np.empty(sum(s for _, s in lst), np.float32)
    _lib().azw_network(*cfg, seed, flat.ctypes.data_as(C.POINTER(C.c_float)))
    out, off = {}, 0
    for name, size in lst:
        out[name] = flat[off:off + size]
        off += size
    return out


def positions(w: Workload, B=None, seed=SEED):
    """(input [B][P][A] float32, legal [B][A+1] uint8)."""
    B = w.batch if B is None else B
    n, H = w.cfg[0], w.cfg[1]
    inp = np.empty((B, 2 * H + 2, n * n), np.float32)
    legal = np.empty((B, n * n + 1), np.uint8)
    _lib().azw_positions(n, H, B, seed, w.tag, w.p_black, w.p_white,
                         inp.ctypes.data_as(C.POINTER(C.c_float)), legal.ctypes.data_as(C.POINTER(C.c_uint8)))
    return inp, legal


def stones(w: Workload, B=None, seed=SEED):
    """The same boards as positions(), as bytes: (stones [B][n*n], to_move [B])."""
    B = w.batch if B is None else B
    n = w.cfg[0]
    st = np.empty((B, n * n), np.uint8)
    tm = np.empty(B, np.uint8)
    _lib().azw_stones(n, B, seed, w.tag, w.p_black, w.p_white, st.ctypes.data_as(C.POINTER(C.c_uint8)),
                      tm.ctypes.data_as(C.POINTER(C.c_uint8)))
    return st, tm
