"""The .azn checkpoint reader of the C ABI (azh_checkpoint_config,
azh_checkpoint_read; host code, no GPU) against checkpoints the reference's
own saveNetwork wrote (tests/golden/gen0_*.azn, src/checkpoint.cpp:84-100):

- the header and every tensor read back bit for bit: the weights are
  Network(cfg, 1)'s (the oracle's init, itself pinned to the reference), the
  batch-norm statistics generation 0's calibration (calibrated_bn.npz);
- the tensor order and sizes are params() then buffers() (src/network.cpp:113-165);
- every malformed file is refused with loadNetwork's message (bad magic,
  unsupported version, bad ownership flag, bad shape, count, name and size
  mismatches, trailing data, truncation at any point, missing file). Where
  the reference's own build is present (oracle/_ref), its loadNetwork reads
  the same mutated bytes and the two messages must be identical.
"""
import os
import struct

import numpy as np
import pytest

import azgo_hip
import oracle as O
from _util import GOLDEN, calibrated_network

V1 = os.path.join(GOLDEN, "gen0_5x5_4x32.azn")
V2 = os.path.join(GOLDEN, "gen0_5x5_2x16_own.azn")
CFG_V1 = O.WORKLOADS[1].cfg
CFG_V2 = O.make_cfg(5, 2, 16, ownership=1)


def _bytes(path):
    with open(path, "rb") as f:
        return f.read()


def _tensor_offsets(data):
    """[(name, name offset, size offset, data offset, size)] of every tensor."""
    version = struct.unpack_from("<I", data, 4)[0]
    off = 8 + 20 + (4 if version == 2 else 0)
    count = struct.unpack_from("<I", data, off)[0]
    off += 4
    out = []
    for _ in range(count):
        n = struct.unpack_from("<I", data, off)[0]
        name = data[off + 4:off + 4 + n].decode()
        size_off = off + 4 + n
        size = struct.unpack_from("<Q", data, size_off)[0]
        out.append((name, off, size_off, size_off + 8, size))
        off = size_off + 8 + 4 * size
    assert off == len(data)
    return out


def _ours(path):
    try:
        azgo_hip.checkpoint_read(path)
    except azgo_hip.HipError as e:
        return e.code, str(e)
    return azgo_hip.OK, ""


def _reference(path, cfg):
    if not O.ref_available():
        return None
    try:
        O.RefNetwork.load_file(path, cfg)
    except RuntimeError as e:
        return str(e)
    return ""


def test_header_of_reference_checkpoints():
    for path, cfg in ((V1, CFG_V1), (V2, CFG_V2)):
        c = azgo_hip.checkpoint_config(path)
        got = (c.board, c.history, c.blocks, c.filters, c.value_hidden, c.ownership)
        assert got == (cfg.board, cfg.history, cfg.blocks, cfg.filters, cfg.value_hidden, cfg.ownership)
    # the version word: 1 without the ownership head, 2 with it (include/azgo/checkpoint.hpp:12-18)
    assert struct.unpack_from("<II", _bytes(V1)) == (0x4F475A41, 1)
    assert struct.unpack_from("<II", _bytes(V2)) == (0x4F475A41, 2)
    assert _bytes(V1)[:4] == b"AZGO"


def test_tensors_read_bitwise():
    cfg, tensors = azgo_hip.checkpoint_read(V1)
    want = calibrated_network("1").tensors()
    assert list(tensors) == list(want)
    for name, t in want.items():
        assert np.array_equal(tensors[name].view(np.uint32), t.view(np.uint32)), name

    cfg, tensors = azgo_hip.checkpoint_read(V2)
    init = O.init_network(CFG_V2, synthetic_bn=False).tensors()
    assert list(tensors) == list(init)
    for name, t in init.items():
        if name.endswith(".runMean") or name.endswith(".runVar"):
            continue   # calibrated: checked for plausibility below
        assert np.array_equal(tensors[name].view(np.uint32), t.view(np.uint32)), name
    for name, t in tensors.items():
        if name.endswith(".runVar"):
            assert (t > 0).all() and np.isfinite(t).all(), name


def test_tensor_spec_is_the_reference_layout():
    for cfg, path in ((CFG_V1, V1), (CFG_V2, V2), (O.WORKLOADS[3].cfg, None), (O.WORKLOADS[5].cfg, None)):
        spec = azgo_hip.tensor_spec(azgo_hip.net_cfg(cfg.board, cfg.history, cfg.blocks, cfg.filters,
                                                     cfg.value_hidden, cfg.ownership))
        assert spec == [(name, size) for name, size, _, _ in O.layout(cfg)]
        if path:   # the file's own order and sizes
            assert [(e[0], e[4]) for e in _tensor_offsets(_bytes(path))] == spec


def _mutations():
    """(label, bytes) of malformed checkpoints built from the version-1 file."""
    data = _bytes(V1)
    ents = _tensor_offsets(data)
    out = []
    out.append(("magic", b"AZGP" + data[4:]))
    out.append(("version 3", data[:4] + struct.pack("<I", 3) + data[8:]))
    out.append(("version 0", data[:4] + struct.pack("<I", 0) + data[8:]))
    out.append(("board 4", data[:8] + struct.pack("<i", 4) + data[12:]))
    out.append(("board 21", data[:8] + struct.pack("<i", 21) + data[12:]))
    out.append(("history 0", data[:12] + struct.pack("<i", 0) + data[16:]))
    out.append(("blocks -1", data[:16] + struct.pack("<i", -1) + data[20:]))
    out.append(("filters 513", data[:20] + struct.pack("<i", 513) + data[24:]))
    out.append(("value 1025", data[:24] + struct.pack("<i", 1025) + data[28:]))
    # version 2 with an ownership flag of 2
    v2 = _bytes(V2)
    out.append(("ownership flag", v2[:28] + struct.pack("<i", 2) + v2[32:]))
    # version 1 header claiming version 2: the tensor count is read as the flag
    out.append(("v1 as v2", data[:4] + struct.pack("<I", 2) + data[8:]))
    # tensor count off by one
    out.append(("count", data[:28] + struct.pack("<I", len(ents) - 1) + data[32:]))
    # a wrong tensor name (same length, so the rest still parses)
    name, noff, _, _, _ = ents[3]
    bad = bytearray(data)
    bad[noff + 4] = ord("X")
    out.append(("name", bytes(bad)))
    # a wrong size field
    _, _, soff, _, size = ents[5]
    out.append(("size", data[:soff] + struct.pack("<Q", size + 1) + data[soff + 8:]))
    # trailing data
    out.append(("trailing", data + b"\0"))
    # truncation inside the header, a name, a size, the floats, at the very end
    for cut in (3, 20, 30, ents[0][1] + 6, ents[2][2] + 3, ents[4][3] + 10, len(data) - 1):
        out.append((f"cut {cut}", data[:cut]))
    out.append(("empty", b""))
    return out


@pytest.mark.parametrize("label,blob", _mutations(), ids=[m[0] for m in _mutations()])
def test_malformed_refused_like_load_network(tmp_path, label, blob):
    path = str(tmp_path / "net.azn")
    with open(path, "wb") as f:
        f.write(blob)
    code, msg = _ours(path)
    assert code == azgo_hip.ERR_FORMAT, (label, code, msg)
    assert msg.startswith(path + ": "), msg
    ref = _reference(path, CFG_V1)
    if ref is not None:
        assert ref == msg, (label, ref, msg)
    # the header-only reader refuses header problems the same way
    if label.startswith(("magic", "version", "board", "history", "blocks", "filters", "value", "ownership")):
        with pytest.raises(azgo_hip.HipError) as e:
            azgo_hip.checkpoint_config(path)
        assert str(e.value) == msg


def test_expected_messages():
    """The wording, independently of the reference build."""
    msgs = {label: _ours_blob(label, blob) for label, blob in _mutations()}
    assert msgs["magic"].endswith(": not an AZGO checkpoint")
    assert msgs["version 3"].endswith(": unsupported version 3")
    assert msgs["board 4"].endswith(": invalid network shape in header")
    assert msgs["ownership flag"].endswith(": invalid ownership flag in header")
    n = len(_tensor_offsets(_bytes(V1)))
    assert msgs["count"].endswith(f": has {n - 1} tensors but the network needs {n}")
    assert "' but expected '" in msgs["name"] and msgs["name"].split(": ", 1)[1].startswith("tensor 3 is '")
    assert msgs["size"].endswith(" values but expected " + str(_tensor_offsets(_bytes(V1))[5][4]))
    assert msgs["trailing"].endswith(": unexpected data after the last tensor")
    assert msgs["empty"].endswith(": truncated") and msgs["cut 20"].endswith(": truncated")


def _ours_blob(label, blob):
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "net.azn")
        with open(path, "wb") as f:
            f.write(blob)
        return _ours(path)[1]


def test_missing_file():
    path = os.path.join(GOLDEN, "no_such_checkpoint.azn")
    code, msg = _ours(path)
    assert code == azgo_hip.ERR_FORMAT and msg == "cannot open checkpoint " + path
    ref = _reference(path, CFG_V1)
    if ref is not None:
        assert ref == msg


def test_read_capacity_checked():
    import ctypes as C
    lib = azgo_hip.load()
    cfg, total = azgo_hip.NetCfg(), C.c_size_t()
    assert lib.azh_checkpoint_read(V1.encode(), C.byref(cfg), None, 0, C.byref(total)) == azgo_hip.OK
    small = np.empty(total.value - 1, np.float32)
    rc = lib.azh_checkpoint_read(V1.encode(), C.byref(cfg), small.ctypes.data_as(C.POINTER(C.c_float)),
                                 small.size, C.byref(total))
    assert rc == azgo_hip.ERR_ARGUMENT
    assert sum(size for _, size, _, _ in O.layout(CFG_V1)) == total.value
