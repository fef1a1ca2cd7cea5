"""Python binding of the MI355X inference backend's C ABI (include/azgo_hip.h).

A thin ctypes layer used by the tests and the benchmark; the product is
libazgo_hip.so, which it loads from this directory. There is no fallback: if
the library is missing, loading raises, and every call that needs the GPU
fails with the library's own error.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libazgo_hip.so")

OK = 0
ERR_ARGUMENT, ERR_UNAVAILABLE, ERR_MEMORY, ERR_TENSOR, ERR_HIP, ERR_STATE, ERR_FORMAT = -1, -2, -3, -4, -5, -6, -7


class NetCfg(C.Structure):
    """azh_netcfg (NetConfig, include/azgo/network.hpp:24-36)."""
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


class Tensor(C.Structure):
    _fields_ = [("name", C.c_char_p), ("data", C.POINTER(C.c_float)), ("size", C.c_size_t)]


class Positions(C.Structure):
    """azh_positions: a batch of positions as MCTS leaves hand them over."""
    _fields_ = [("stones", C.POINTER(C.c_uint8)), ("plies", C.POINTER(C.c_int32)),
                ("to_move", C.POINTER(C.c_uint8)), ("sym", C.POINTER(C.c_uint8)),
                ("seen", C.POINTER(C.c_uint64)), ("seen_offsets", C.POINTER(C.c_int64))]


class HubGroup(C.Structure):
    """azh_hub_group: GpuHubs (include/azgo/gpu_memory.hpp)."""
    _fields_ = [("hubs", C.c_int), ("slots_per_hub", C.c_int), ("max_batch", C.c_int)]


DONE_FN = C.CFUNCTYPE(None, C.c_void_p, C.c_int, C.c_char_p)


class HipError(RuntimeError):
    def __init__(self, code, message):
        super().__init__(message)
        self.code = code


def load():
    """The native library, loaded once. Raises if it is not built."""
    if not hasattr(load, "lib"):
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"azgo_hip: native library missing: {LIB_PATH} (build it with "
                               f"alphazero-go_amd/build.py)")
        h = C.CDLL(LIB_PATH)
        P = C.POINTER
        f32, u8, vp = P(C.c_float), P(C.c_uint8), C.c_void_p
        sig = {
            "azh_built": ([], C.c_int),
            "azh_available": ([C.c_char_p, C.c_size_t], C.c_int),
            "azh_describe": ([C.c_char_p, C.c_size_t], C.c_int),
            "azh_device_cus": ([P(C.c_int)], C.c_int),
            "azh_last_error": ([], C.c_char_p),
            "azh_memory_need": ([P(NetCfg), C.c_int, C.c_int, P(C.c_size_t)], C.c_int),
            "azh_check_memory": ([P(NetCfg), C.c_int, C.c_int, C.c_int], C.c_int),
            "azh_check_memory_groups": ([P(NetCfg), P(HubGroup), C.c_int], C.c_int),
            "azh_create": ([P(NetCfg), P(Tensor), C.c_int, C.c_int, C.c_int, P(vp)], C.c_int),
            "azh_tensor_count": ([P(NetCfg), P(C.c_int)], C.c_int),
            "azh_tensor_info": ([P(NetCfg), C.c_int, C.c_char_p, C.c_size_t, P(C.c_size_t)], C.c_int),
            "azh_checkpoint_config": ([C.c_char_p, P(NetCfg)], C.c_int),
            "azh_checkpoint_read": ([C.c_char_p, P(NetCfg), f32, C.c_size_t, P(C.c_size_t)], C.c_int),
            "azh_create_from_checkpoint": ([C.c_char_p, C.c_int, C.c_int, P(vp)], C.c_int),
            "azh_destroy": ([vp], None),
            "azh_slots": ([vp], C.c_int),
            "azh_max_batch": ([vp], C.c_int),
            "azh_slot_input": ([vp, C.c_int], f32),
            "azh_slot_logits": ([vp, C.c_int], f32),
            "azh_slot_values": ([vp, C.c_int], f32),
            "azh_begin": ([vp, C.c_int, C.c_int, DONE_FN, vp], C.c_int),
            "azh_infer": ([vp, f32, C.c_int, f32, f32, f32], C.c_int),
            "azh_infer_noalloc": ([vp, vp, C.c_int, vp, vp, vp, vp], C.c_int),
            "azh_softmax_legal": ([f32, u8, C.c_int, C.c_int, f32], C.c_int),
            "azh_encode_planes": ([u8, P(C.c_int32), u8, u8, C.c_int, C.c_int, C.c_int, f32], C.c_int),
            "azh_legal_moves": ([u8, C.c_int, u8, P(C.c_uint64), P(C.c_int64), C.c_int, u8], C.c_int),
            "azh_evaluate_positions": ([vp, P(Positions), C.c_int, f32, f32, u8, f32], C.c_int),
            "azh_time_positions": ([vp, P(Positions), C.c_int, C.c_int, f32], C.c_int),
            "azh_begin_positions": ([vp, C.c_int, C.c_int, P(Positions), DONE_FN, vp], C.c_int),
            "azh_slot_position_logits": ([vp, C.c_int], f32),
            "azh_slot_priors": ([vp, C.c_int], f32),
            "azh_slot_legal": ([vp, C.c_int], u8),
            "azh_time_pipelined_positions": ([vp, P(Positions), C.c_int, C.c_int, f32], C.c_int),
            "azh_set_graphs": ([vp, C.c_int], C.c_int),
            "azh_set_small_tower": ([vp, C.c_int], C.c_int),
            "azh_set_resident_tower": ([vp, C.c_int], C.c_int),
            "azh_time_resident_tower": ([vp, C.c_int, C.c_int, C.c_int, C.c_int, f32], C.c_int),
            "azh_pass_form": ([vp, C.c_int, C.c_int, P(C.c_int)], C.c_int),
            "azh_stage": ([vp, C.c_int, C.c_int], C.c_int),
            "azh_enqueue": ([vp, C.c_int, C.c_int], C.c_int),
            "azh_synchronize": ([vp, C.c_int], C.c_int),
            "azh_fetch": ([vp, C.c_int, C.c_int], C.c_int),
            "azh_time_passes": ([vp, C.c_int, C.c_int, C.c_int, f32], C.c_int),
            "azh_time_tower_convs": ([vp, C.c_int, C.c_int, C.c_int, f32, P(C.c_int), P(C.c_int)], C.c_int),
            "azh_time_round_trips": ([vp, C.c_int, C.c_int, C.c_int, f32], C.c_int),
            "azh_time_tower_layers": ([vp, C.c_int, C.c_int, C.c_int, f32, P(C.c_int)], C.c_int),
            "azh_time_pipelined": ([vp, C.c_int, C.c_int, f32], C.c_int),
            "azh_probe_conv3x3": ([f32, f32, f32, f32, f32, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                   f32], C.c_int),
            "azh_time_conv3x3": ([C.c_int] * 6 + [f32], C.c_int),
            "azh_probe_heads": ([vp, f32, C.c_int, f32, f32, f32], C.c_int),
            "azh_probe_trunk": ([vp, f32, C.c_int, C.c_int, f32], C.c_int),
            "azh_probe_fill": ([f32, C.c_size_t, C.c_float, C.c_size_t], C.c_int),
            "azh_probe_copy": ([C.c_size_t, C.c_int, f32], C.c_int),
            "azh_probe_mfma": ([C.c_int, C.c_int, f32, P(C.c_double)], C.c_int),
            "azh_set_hub_chaos_seed": ([C.c_uint64], None),
            "azh_hub_chaos_seed": ([], C.c_uint64),
            "azh_fail_passes_after": ([C.c_int], None),
            "azh_set_memory_limit": ([C.c_size_t], None),
            "azh_passes_completed": ([], C.c_longlong),
            "azh_set_copy_out_delay": ([C.c_int], None),
        }
        for name, (args, res) in sig.items():
            fn = getattr(h, name)
            fn.argtypes = args
            fn.restype = res
        load.lib = h
        load.symbols = sorted(sig)
    return load.lib


def _check(rc):
    if rc != OK:
        raise HipError(rc, load().azh_last_error().decode())


def _f(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def available():
    """(usable, why)."""
    buf = C.create_string_buffer(512)
    ok = load().azh_available(buf, 512)
    return bool(ok), buf.value.decode()


def describe():
    buf = C.create_string_buffer(512)
    _check(load().azh_describe(buf, 512))
    return buf.value.decode()


def device_cus():
    """The device's compute units, as the runner's launch rules count them."""
    n = C.c_int()
    _check(load().azh_device_cus(C.byref(n)))
    return n.value


def net_cfg(board, history, blocks, filters, value_hidden, ownership=0):
    return NetCfg(board, history, blocks, filters, value_hidden, ownership)


def memory_need(cfg, max_batch, slots):
    n = C.c_size_t()
    _check(load().azh_memory_need(C.byref(cfg), max_batch, slots, C.byref(n)))
    return n.value


def check_memory(cfg, max_batch, hubs, slots_per_hub=2):
    _check(load().azh_check_memory(C.byref(cfg), max_batch, hubs, slots_per_hub))


def check_memory_groups(cfg, groups):
    """groups: (hubs, slots_per_hub, max_batch) triples, summed as one check."""
    arr = (HubGroup * max(1, len(groups)))(*[HubGroup(*g) for g in groups])
    _check(load().azh_check_memory_groups(C.byref(cfg), arr, len(groups)))


def _u8(a):
    return None if a is None else a.ctypes.data_as(C.POINTER(C.c_uint8))


def _seen_lists(seen, B):
    """[list of uint64 hashes per position] -> (concatenated, offsets [B+1])."""
    if seen is None:
        seen = [()] * B
    if len(seen) != B:
        raise ValueError("one seen list per position")
    offs = np.zeros(B + 1, np.int64)
    for b, lst in enumerate(seen):
        offs[b + 1] = offs[b] + len(lst)
    flat = np.zeros(max(1, int(offs[-1])), np.uint64)
    if offs[-1]:
        flat[:offs[-1]] = np.concatenate([np.asarray(x, np.uint64).reshape(-1) for x in seen])
    return flat, offs


def encode_planes(stones, to_move, n, H, plies=None, sym=None):
    """stones [B][H][n*n] bytes -> planes [B][2H+2][n*n] (azh_encode_planes)."""
    stones = np.ascontiguousarray(stones, np.uint8)
    B = stones.shape[0]
    to_move = np.ascontiguousarray(to_move, np.uint8)
    pl = None if plies is None else np.ascontiguousarray(plies, np.int32)
    sy = None if sym is None else np.ascontiguousarray(sym, np.uint8)
    out = np.empty((B, 2 * H + 2, n * n), np.float32)
    _check(load().azh_encode_planes(_u8(stones), None if pl is None else pl.ctypes.data_as(C.POINTER(C.c_int32)),
                                    _u8(to_move), _u8(sy), B, n, H, _f(out)))
    return out


def legal_moves(stones, to_move, n, seen=None):
    """stones [B][n*n], to_move [B], seen: per position a list of hashes ->
    legal [B][n*n+1] (azh_legal_moves)."""
    stones = np.ascontiguousarray(stones, np.uint8).reshape(-1, n * n)
    B = stones.shape[0]
    to_move = np.ascontiguousarray(to_move, np.uint8)
    flat, offs = _seen_lists(seen, B)
    out = np.empty((B, n * n + 1), np.uint8)
    _check(load().azh_legal_moves(_u8(stones), n, _u8(to_move), flat.ctypes.data_as(C.POINTER(C.c_uint64)),
                                  offs.ctypes.data_as(C.POINTER(C.c_int64)), B, _u8(out)))
    return out


def tensor_spec(cfg):
    """[(name, floats)] of the network's params() then buffers()."""
    lib = load()
    n = C.c_int()
    _check(lib.azh_tensor_count(C.byref(cfg), C.byref(n)))
    out = []
    name = C.create_string_buffer(128)
    size = C.c_size_t()
    for i in range(n.value):
        _check(lib.azh_tensor_info(C.byref(cfg), i, name, 128, C.byref(size)))
        out.append((name.value.decode(), size.value))
    return out


def checkpoint_config(path):
    """The NetCfg in an .azn checkpoint's header."""
    cfg = NetCfg()
    _check(load().azh_checkpoint_config(os.fsencode(path), C.byref(cfg)))
    return cfg


def checkpoint_read(path):
    """(cfg, {name: float32 array}) from an .azn checkpoint, checked as
    loadNetwork checks it."""
    lib = load()
    cfg, total = NetCfg(), C.c_size_t()
    _check(lib.azh_checkpoint_read(os.fsencode(path), C.byref(cfg), None, 0, C.byref(total)))
    values = np.empty(total.value, np.float32)
    _check(lib.azh_checkpoint_read(os.fsencode(path), C.byref(cfg), _f(values), values.size, C.byref(total)))
    tensors, off = {}, 0
    for name, size in tensor_spec(cfg):
        tensors[name] = values[off:off + size]
        off += size
    return cfg, tensors


class Runner:
    """An azh_runner: the network's weights on the GPU, `slots` slots of up to
    max_batch positions. tensors: {name: float array} of the network's
    params() and buffers()."""

    def __init__(self, cfg: NetCfg, tensors: dict, max_batch: int, slots: int = 2):
        self.lib = load()
        self.cfg = cfg
        arrays = [(k.encode(), _f32(v)) for k, v in tensors.items()]
        table = (Tensor * len(arrays))()
        for i, (k, v) in enumerate(arrays):
            table[i] = Tensor(k, _f(v), v.size)
        h = C.c_void_p()
        _check(self.lib.azh_create(C.byref(cfg), table, len(arrays), max_batch, slots, C.byref(h)))
        self.h = h
        self.max_batch = max_batch
        self._callbacks = {}

    @classmethod
    def from_checkpoint(cls, path, max_batch, slots=2):
        """A runner straight from an .azn checkpoint (azh_create_from_checkpoint)."""
        self = cls.__new__(cls)
        self.lib = load()
        self.cfg = checkpoint_config(path)
        h = C.c_void_p()
        _check(self.lib.azh_create_from_checkpoint(os.fsencode(path), max_batch, slots, C.byref(h)))
        self.h = h
        self.max_batch = max_batch
        self._callbacks = {}
        return self

    def close(self):
        if getattr(self, "h", None):
            self.lib.azh_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    @property
    def slots(self):
        return self.lib.azh_slots(self.h)

    def infer(self, inp, ownership=False):
        """(logits, values), plus ownership [B][area] when asked."""
        inp = _f32(inp)
        B = inp.shape[0]
        logits = np.empty((B, self.cfg.actions), np.float32)
        values = np.empty(B, np.float32)
        own = np.empty((B, self.cfg.board * self.cfg.board), np.float32) if ownership else None
        _check(self.lib.azh_infer(self.h, _f(inp), B, _f(logits), _f(values), _f(own) if ownership else None))
        return (logits, values, own) if ownership else (logits, values)

    def _positions(self, stones, to_move, plies, sym, seen):
        stones = np.ascontiguousarray(stones, np.uint8)
        B = stones.shape[0]
        keep = [stones, np.ascontiguousarray(to_move, np.uint8),
                None if plies is None else np.ascontiguousarray(plies, np.int32),
                None if sym is None else np.ascontiguousarray(sym, np.uint8)]
        flat, offs = _seen_lists(seen, B)
        keep += [flat, offs]
        pos = Positions(_u8(keep[0]), None if keep[2] is None else keep[2].ctypes.data_as(C.POINTER(C.c_int32)),
                        _u8(keep[1]), _u8(keep[3]), flat.ctypes.data_as(C.POINTER(C.c_uint64)),
                        offs.ctypes.data_as(C.POINTER(C.c_int64)))
        return B, pos, keep

    def time_positions(self, stones, to_move, plies=None, sym=None, seen=None, iters=10):
        """Total ms of `iters` runs of each step: (encode, legal, priors, whole chain)."""
        B, pos, keep = self._positions(stones, to_move, plies, sym, seen)
        ms = (C.c_float * 4)()
        _check(self.lib.azh_time_positions(self.h, C.byref(pos), B, iters, ms))
        return tuple(ms)

    def evaluate_positions(self, stones, to_move, plies=None, sym=None, seen=None):
        """The leaf evaluation on the GPU (azh_evaluate_positions): stones
        [B][H][area] bytes -> (logits mapped back, priors, legal, values)."""
        B, pos, keep = self._positions(stones, to_move, plies, sym, seen)
        A1 = self.cfg.actions
        logits = np.empty((B, A1), np.float32)
        priors = np.empty((B, A1), np.float32)
        legal = np.empty((B, A1), np.uint8)
        values = np.empty(B, np.float32)
        _check(self.lib.azh_evaluate_positions(self.h, C.byref(pos), B, _f(logits), _f(priors), _u8(legal),
                                               _f(values)))
        return logits, priors, legal, values

    def begin_positions(self, slot, done, stones, to_move, plies=None, sym=None, seen=None):
        """azh_begin_positions: done(slot, error_or_None) from the completion
        thread; then position_outputs(slot, B) holds the results."""
        B, pos, keep = self._positions(stones, to_move, plies, sym, seen)
        key = (slot, threading.get_ident(), len(self._callbacks))

        def cb(user, s, err):
            done(s, err.decode() if err else None)

        fn = DONE_FN(cb)
        self._callbacks[key] = fn   # kept alive until the runner goes (the positions are copied before the return)
        _check(self.lib.azh_begin_positions(self.h, slot, B, C.byref(pos), fn, None))

    def position_outputs(self, slot, B):
        """(logits mapped back, priors, legal, values) of the slot's last
        begin_positions of B positions."""
        A1 = self.cfg.actions
        out = []
        for fn, dt in ((self.lib.azh_slot_position_logits, np.float32), (self.lib.azh_slot_priors, np.float32),
                       (self.lib.azh_slot_legal, np.uint8)):
            p = fn(self.h, slot)
            if not p:
                raise HipError("no positions pass on this slot")
            out.append(np.ctypeslib.as_array(p, (B * A1,)).reshape(B, A1).astype(dt, copy=True))
        out.append(self.values(slot, B))
        return tuple(out)

    def time_pipelined_positions(self, B, passes, stones, to_move, plies=None, sym=None, seen=None):
        """Wall ms for `passes` positions passes of B with every slot kept
        full through begin_positions (the same positions each time)."""
        n, pos, keep = self._positions(stones, to_move, plies, sym, seen)
        assert n == B
        ms = C.c_float()
        _check(self.lib.azh_time_pipelined_positions(self.h, C.byref(pos), B, passes, C.byref(ms)))
        return ms.value

    def set_graphs(self, enabled):
        _check(self.lib.azh_set_graphs(self.h, int(enabled)))

    def set_small_tower(self, enabled):
        _check(self.lib.azh_set_small_tower(self.h, int(enabled)))

    def set_resident_tower(self, mode):
        """0: per-layer launches; 1: the board-resident tower for a pass alone
        whose batch fills its rounds of CUs (default); 2: wherever the network
        allows it."""
        _check(self.lib.azh_set_resident_tower(self.h, int(mode)))

    # ---- slot staging (the hub's view)
    def input(self, slot):
        p = self.lib.azh_slot_input(self.h, slot)
        n = self.max_batch * self.cfg.planes * self.cfg.area
        return np.ctypeslib.as_array(p, (n,)).reshape(self.max_batch, self.cfg.planes, self.cfg.area)

    def logits(self, slot, B):
        p = self.lib.azh_slot_logits(self.h, slot)
        return np.ctypeslib.as_array(p, (self.max_batch * self.cfg.actions,)).reshape(
            self.max_batch, self.cfg.actions)[:B].copy()

    def values(self, slot, B):
        p = self.lib.azh_slot_values(self.h, slot)
        return np.ctypeslib.as_array(p, (self.max_batch,))[:B].copy()

    def begin(self, slot, B, done):
        """done(slot, error_or_None) from the completion thread."""
        key = (slot, threading.get_ident(), len(self._callbacks))

        def cb(user, s, err, _key=key):
            try:
                done(s, err.decode() if err else None)
            finally:
                pass

        fn = DONE_FN(cb)
        self._callbacks[key] = fn   # kept alive until the runner goes
        _check(self.lib.azh_begin(self.h, slot, B, fn, None))

    # ---- device-resident passes
    def stage(self, slot, B):
        _check(self.lib.azh_stage(self.h, slot, B))

    def enqueue(self, slot, B):
        _check(self.lib.azh_enqueue(self.h, slot, B))

    def synchronize(self, slot):
        _check(self.lib.azh_synchronize(self.h, slot))

    def fetch(self, slot, B):
        _check(self.lib.azh_fetch(self.h, slot, B))
        return self.logits(slot, B), self.values(slot, B)

    def time_passes(self, slot, B, iters):
        ms = C.c_float()
        _check(self.lib.azh_time_passes(self.h, slot, B, iters, C.byref(ms)))
        return ms.value

    def time_tower_convs(self, slot, B, iters):
        """(total ms, launches, layers) of `iters` runs of the tower."""
        ms = C.c_float()
        n, layers = C.c_int(), C.c_int()
        _check(self.lib.azh_time_tower_convs(self.h, slot, B, iters, C.byref(ms), C.byref(n), C.byref(layers)))
        return ms.value, n.value, layers.value

    def time_tower_layers(self, slot, B, iters):
        """(total ms, layers) of `iters` runs of the tower as the pass runs it."""
        ms, layers = C.c_float(), C.c_int()
        _check(self.lib.azh_time_tower_layers(self.h, slot, B, iters, C.byref(ms), C.byref(layers)))
        return ms.value, layers.value

    def time_resident_tower(self, slot, B, iters, stem=True):
        """Total ms of `iters` board-resident launches over B boards (the stem
        first when asked, as a pass runs it)."""
        ms = C.c_float()
        _check(self.lib.azh_time_resident_tower(self.h, slot, B, iters, int(stem), C.byref(ms)))
        return ms.value

    # azh_pass_form's mask bits
    FORM_SMALL, FORM_RESIDENT, FORM_SPLIT = 1, 2, 4

    def pass_form(self, B, alone=True):
        """How a pass of B runs: a mask of FORM_SMALL, FORM_RESIDENT, FORM_SPLIT."""
        form = C.c_int()
        _check(self.lib.azh_pass_form(self.h, B, int(alone), C.byref(form)))
        return form.value

    def time_round_trips(self, slot, B, iters):
        ms = C.c_float()
        _check(self.lib.azh_time_round_trips(self.h, slot, B, iters, C.byref(ms)))
        return ms.value

    def time_pipelined(self, B, passes):
        """Wall ms for `passes` passes of B with every slot kept full
        through begin/done (each slot's input must hold B positions)."""
        ms = C.c_float()
        _check(self.lib.azh_time_pipelined(self.h, B, passes, C.byref(ms)))
        return ms.value

    # ---- probes
    def probe_heads(self, trunk, ownership=False):
        trunk = _f32(trunk)
        B = trunk.shape[0]
        logits = np.empty((B, self.cfg.actions), np.float32)
        values = np.empty(B, np.float32)
        own = np.empty((B, self.cfg.board * self.cfg.board), np.float32) if ownership else None
        _check(self.lib.azh_probe_heads(self.h, _f(trunk), B, _f(logits), _f(values), _f(own) if ownership else None))
        return (logits, values, own) if ownership else (logits, values)

    def infer_noalloc(self, d_input, B, d_logits, d_values, d_ownership=None, stream=None):
        """The pass on device arrays (integer device addresses) enqueued on
        `stream` (an integer hipStream_t, None: the null stream), allocating
        nothing; the caller synchronizes."""
        _check(self.lib.azh_infer_noalloc(self.h, C.c_void_p(d_input), B, C.c_void_p(d_logits),
                                          C.c_void_p(d_values), C.c_void_p(d_ownership) if d_ownership else None,
                                          C.c_void_p(stream) if stream else None))

    def probe_trunk(self, inp, blocks):
        inp = _f32(inp)
        B = inp.shape[0]
        out = np.empty((B, self.cfg.filters, self.cfg.area), np.float32)
        _check(self.lib.azh_probe_trunk(self.h, _f(inp), B, blocks, _f(out)))
        return out


def softmax_legal(logits, legal):
    logits = _f32(logits)
    legal = np.ascontiguousarray(legal, np.uint8)
    B, A1 = logits.shape
    out = np.empty_like(logits)
    _check(load().azh_softmax_legal(_f(logits), legal.ctypes.data_as(C.POINTER(C.c_uint8)), B, A1, _f(out)))
    return out


def probe_conv3x3(x, w, scale, shift, skip=None, relu=True, tiling=-1):
    """x [B][cin][n*n], w [cout][cin*9] -> y [B][cout][n*n]."""
    x = _f32(x)
    w = _f32(w)
    B, cin, A = x.shape
    n = int(round(A ** 0.5))
    cout = w.shape[0]
    y = np.empty((B, cout, A), np.float32)
    sk = _f32(skip) if skip is not None else None
    _check(load().azh_probe_conv3x3(_f(x), _f(w), _f(_f32(scale)), _f(_f32(shift)),
                                    _f(sk) if sk is not None else None, int(relu), B, n, cin, cout, tiling, _f(y)))
    return y


def time_conv3x3(B, n, cin, cout, tiling=-1, iters=10):
    """Average ms of one 3x3 convolution launch (device-resident data)."""
    ms = C.c_float()
    _check(load().azh_time_conv3x3(B, n, cin, cout, tiling, iters, C.byref(ms)))
    return ms.value / iters


def probe_fill(data, n, value, tail=0):
    data = _f32(data).copy()
    _check(load().azh_probe_fill(_f(data), n, value, tail))
    return data


def probe_mfma(chain, iters):
    """(total ms, flops per launch) of `iters` launches of dependent MFMA
    chains, one 8-wave workgroup per CU."""
    ms, flops = C.c_float(), C.c_double()
    _check(load().azh_probe_mfma(chain, iters, C.byref(ms), C.byref(flops)))
    return ms.value, flops.value


def probe_copy(nbytes, iters):
    ms = C.c_float()
    _check(load().azh_probe_copy(nbytes, iters, C.byref(ms)))
    return ms.value


def set_hub_chaos_seed(seed):
    load().azh_set_hub_chaos_seed(seed)


def hub_chaos_seed():
    return load().azh_hub_chaos_seed()


def fail_passes_after(n):
    load().azh_fail_passes_after(n)


def set_memory_limit(nbytes):
    load().azh_set_memory_limit(nbytes)


def passes_completed():
    return load().azh_passes_completed()


def set_copy_out_delay(us):
    load().azh_set_copy_out_delay(us)


def exported_symbols():
    """The C ABI's symbols this binding declares (include/azgo_hip.h)."""
    load()
    return list(load.symbols)
