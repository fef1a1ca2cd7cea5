"""azh_infer_noalloc: azh_infer's pass on device arrays, allocating nothing
(its intermediates live in the library's static scratch array), enqueued on
a caller's stream. Checked against azh_infer, the entry point it varies, on
the same positions: the same kernels, so the same bits, for logits, values
and ownership; two calls in a row on the same stream, the second with a
smaller batch (the scratch keeps the first call's contents); the
small-board one-launch pass and the per-layer launches; the call captured
into a HIP graph on the caller's stream (global capture mode, so any
allocation or synchronizing call on its path would fail the capture) and the
graph launched twice, each launch equal to azh_infer; and a batch above the
scratch array's capacity refused before anything runs.

The test allocates its device arrays and stream through the HIP runtime
(the entry point never does).
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from _util import bitwise_equal, to_hip_cfg

pytestmark = pytest.mark.gpu

H2D, D2H = 1, 2


class Hip:
    """The HIP runtime calls the test itself makes (device arrays, a stream)."""

    def __init__(self):
        self.lib = C.CDLL("/opt/rocm/lib/libamdhip64.so")
        self.lib.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.lib.hipFree.argtypes = [C.c_void_p]
        self.lib.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.lib.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.lib.hipStreamSynchronize.argtypes = [C.c_void_p]
        self.lib.hipStreamDestroy.argtypes = [C.c_void_p]
        self.lib.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
        self.lib.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
        self.lib.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p,
                                                 C.c_size_t]
        self.lib.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
        self.lib.hipGraphExecDestroy.argtypes = [C.c_void_p]
        self.lib.hipGraphDestroy.argtypes = [C.c_void_p]
        self.held = []

    def ok(self, rc, what):
        assert rc == 0, f"{what} returned {rc}"

    def alloc(self, nbytes):
        p = C.c_void_p()
        self.ok(self.lib.hipMalloc(C.byref(p), nbytes), "hipMalloc")
        self.held.append(p.value)
        return p.value

    def upload(self, a):
        a = np.ascontiguousarray(a)
        d = self.alloc(a.nbytes)
        self.ok(self.lib.hipMemcpy(d, a.ctypes.data, a.nbytes, H2D), "hipMemcpy")
        return d

    def filled(self, shape, value=np.nan):
        return self.upload(np.full(shape, value, np.float32))

    def download(self, d, shape):
        out = np.empty(shape, np.float32)
        self.ok(self.lib.hipMemcpy(out.ctypes.data, d, out.nbytes, D2H), "hipMemcpy")
        return out

    def stream(self):
        s = C.c_void_p()
        self.ok(self.lib.hipStreamCreate(C.byref(s)), "hipStreamCreate")
        return s.value

    def close(self, stream=None):
        if stream:
            self.ok(self.lib.hipStreamSynchronize(stream), "hipStreamSynchronize")
            self.lib.hipStreamDestroy(stream)
        for p in self.held:
            self.lib.hipFree(p)
        self.held = []


def _noalloc(hip_rt, r, cfg, inp, stream, ownership=False):
    B = inp.shape[0]
    d_in = hip_rt.upload(inp.astype(np.float32))
    d_l = hip_rt.filled((B, cfg.actions))
    d_v = hip_rt.filled((B,))
    d_o = hip_rt.filled((B, cfg.area)) if ownership else None
    r.infer_noalloc(d_in, B, d_l, d_v, d_o, stream)
    hip_rt.ok(hip_rt.lib.hipStreamSynchronize(stream), "hipStreamSynchronize")
    out = [hip_rt.download(d_l, (B, cfg.actions)), hip_rt.download(d_v, (B,))]
    if ownership:
        out.append(hip_rt.download(d_o, (B, cfg.area)))
    return out


# (network, first batch, second batch, ownership): the 19x19 10x128
# benchmark network through the per-layer launches, a 19x19 128-channel
# network through the board-resident tower at 256 boards (then per layer at
# 13), the 5x5 one through the one-launch small-board pass, a 9x9 network
# with the ownership head.
CASES = [
    ("19x19 10x128", lambda: O.init_network(O.WORKLOADS[3].cfg), O.WORKLOADS[3], 48, 13, False),
    ("19x19 2x128 resident", lambda: O.random_network(O.make_cfg(19, 2, 128), 72), O.WORKLOADS[3], 256, 13, False),
    ("5x5 4x32", lambda: O.init_network(O.WORKLOADS[1].cfg), O.WORKLOADS[1], 8, 3, False),
    ("9x9 2x16 own", lambda: O.random_network(O.make_cfg(9, 2, 16, value_hidden=16, ownership=1), 71),
     O.WORKLOADS[2], 6, 2, True),
]


@pytest.mark.parametrize("name,make,w,B1,B2,own", CASES, ids=[c[0] for c in CASES])
def test_noalloc_equals_infer(hip, name, make, w, B1, B2, own):
    net = make()
    cfg = net.cfg
    inp, _ = O.workload_inputs(O.Workload(w.tag, w.name, cfg, B1, w.p_black, w.p_white), B1)
    print(f"{name}: azh_infer_noalloc at B={B1} then B={B2}", flush=True)
    rt = Hip()
    stream = rt.stream()
    try:
        with hip.Runner(to_hip_cfg(hip, cfg), net.tensors(), B1, 1) as r:
            for B in (B1, B2):
                want = r.infer(inp[:B], ownership=own)
                got = _noalloc(rt, r, cfg, inp[:B], stream, ownership=own)
                assert np.isfinite(got[0]).all() and np.isfinite(got[1]).all(), (name, B)
                for g, e in zip(got, want):
                    assert bitwise_equal(g, e), (name, B)
    finally:
        rt.close(stream)


def test_noalloc_refuses_beyond_scratch(hip):
    """The 19x19 20x256 network's trunk is 370 KB per board per buffer: 200
    boards need more than the 96 MiB array, refused with the most one call
    takes; a batch within it then runs (on the null stream)."""
    w = O.WORKLOADS[5]
    net = O.init_network(w.cfg)
    rt = Hip()
    try:
        with hip.Runner(to_hip_cfg(hip, w.cfg), net.tensors(), 1, 1) as r:
            with pytest.raises(hip.HipError) as e:
                r.infer_noalloc(1, 200, 1, 1, None, None)   # refused before any pointer is used
            assert e.value.code == hip.ERR_ARGUMENT and "at most" in str(e.value), str(e.value)
            most = int(str(e.value).split("at most ")[1].split()[0])
            assert 100 <= most < 200, most
            inp, _ = O.workload_inputs(w, 2)
            want = r.infer(inp[:1])
            d_in = rt.upload(inp[:1])
            d_l, d_v = rt.filled((1, w.cfg.actions)), rt.filled((1,))
            r.infer_noalloc(d_in, 1, d_l, d_v, None, None)
            rt.ok(rt.lib.hipStreamSynchronize(None), "hipStreamSynchronize")
            assert bitwise_equal(rt.download(d_l, (1, w.cfg.actions)), want[0])
            assert bitwise_equal(rt.download(d_v, (1,)), want[1])
    finally:
        rt.close()


# Captured with hipStreamCaptureModeGlobal: a call on the entry point's path
# that allocates or synchronizes would end the capture with an error.
CAPTURE_GLOBAL = 0


@pytest.mark.parametrize("name,make,w,B1,B2,own", CASES, ids=[c[0] for c in CASES])
def test_noalloc_under_graph_capture(hip, name, make, w, B1, B2, own):
    """azh_infer_noalloc as a caller under HIP graph capture uses it: begin
    capture on the caller's stream, the call, end capture, instantiate, then
    two launches of the graph, each output equal to azh_infer's bits. The
    input changes between the launches (the second batch's positions copied
    over the first's), so the second launch cannot pass on stale outputs."""
    net = make()
    cfg = net.cfg
    inp, _ = O.workload_inputs(O.Workload(w.tag, w.name, cfg, B1, w.p_black, w.p_white), B1)
    other, _ = O.workload_inputs(O.Workload(w.tag + 1, w.name, cfg, B1, w.p_black, w.p_white), B1)
    print(f"{name}: azh_infer_noalloc captured at B={B1}", flush=True)
    rt = Hip()
    stream = rt.stream()
    graph, exe = C.c_void_p(), C.c_void_p()
    try:
        with hip.Runner(to_hip_cfg(hip, cfg), net.tensors(), B1, 1) as r:
            wants = [r.infer(x, ownership=own) for x in (inp, other)]
            d_in = rt.upload(inp.astype(np.float32))
            d_l, d_v = rt.filled((B1, cfg.actions)), rt.filled((B1,))
            d_o = rt.filled((B1, cfg.area)) if own else None
            rt.ok(rt.lib.hipStreamBeginCapture(stream, CAPTURE_GLOBAL), "hipStreamBeginCapture")
            try:
                r.infer_noalloc(d_in, B1, d_l, d_v, d_o, stream)
            finally:
                rt.ok(rt.lib.hipStreamEndCapture(stream, C.byref(graph)), "hipStreamEndCapture")
            rt.ok(rt.lib.hipGraphInstantiate(C.byref(exe), graph, None, None, 0), "hipGraphInstantiate")
            for x, want in zip((inp, other), wants):
                a = np.ascontiguousarray(x, np.float32)
                rt.ok(rt.lib.hipMemcpy(d_in, a.ctypes.data, a.nbytes, H2D), "hipMemcpy")
                rt.ok(rt.lib.hipGraphLaunch(exe, stream), "hipGraphLaunch")
                rt.ok(rt.lib.hipStreamSynchronize(stream), "hipStreamSynchronize")
                got = [rt.download(d_l, (B1, cfg.actions)), rt.download(d_v, (B1,))]
                if own:
                    got.append(rt.download(d_o, (B1, cfg.area)))
                for g, e in zip(got, want):
                    assert bitwise_equal(g, e), name
    finally:
        if exe.value:
            rt.lib.hipGraphExecDestroy(exe)
        if graph.value:
            rt.lib.hipGraphDestroy(graph)
        rt.close(stream)
