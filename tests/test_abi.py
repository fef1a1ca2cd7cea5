"""The C ABI library without a GPU: it loads, exports every function
include/azgo_hip.h declares, and its host-side logic (config validation, the
upload contract, memory arithmetic, test hooks) behaves as the reference's
CUDA backend does. No kernel runs here."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import azgo_hip
import oracle as O
from _util import to_hip_cfg

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "azgo_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(azh_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_function():
    lib = azgo_hip.load()
    names = declared_functions()
    assert len(names) >= 30
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(azgo_hip.exported_symbols()) == names   # the binding declares exactly the header's set


def test_built_and_describe_without_gpu_is_an_answer():
    lib = azgo_hip.load()
    assert lib.azh_built() == 1
    ok, why = azgo_hip.available()
    if not ok:
        assert why   # a reason, never an empty refusal
        with pytest.raises(azgo_hip.HipError) as e:
            azgo_hip.check_memory(to_hip_cfg(azgo_hip, O.WORKLOADS[1].cfg), 8, 1)
        assert e.value.code == azgo_hip.ERR_UNAVAILABLE
        with pytest.raises(azgo_hip.HipError) as e:
            azgo_hip.device_cus()
        assert e.value.code == azgo_hip.ERR_UNAVAILABLE
    else:
        assert azgo_hip.device_cus() > 0


def test_memory_need_formula():
    """Per slot: input, two trunk buffers, the heads' 3 planes, logits,
    values (256-byte aligned); plus the packed weights once."""
    cfg = to_hip_cfg(azgo_hip, O.WORKLOADS[3].cfg)
    one = azgo_hip.memory_need(cfg, 256, 1)
    two = azgo_hip.memory_need(cfg, 256, 2)
    slot = two - one
    al = lambda f: (f + 63) // 64 * 64   # noqa: E731
    B, P, A, F = 256, 18, 361, 128
    assert slot == 4 * (al(B * P * A) + 2 * al(B * F * A) + al(B * 3 * A) + al(B * (A + 1)) + al(B))
    weights = one - slot
    assert 13e6 < weights < 16e6   # ~3.27 M parameters, packed with channel padding


@pytest.mark.parametrize("bad", [
    dict(board=7), dict(board=19, history=0), dict(filters=0), dict(value_hidden=300), dict(blocks=-1),
])
def test_config_validation(bad):
    base = dict(board=9, history=8, blocks=2, filters=16, value_hidden=8, ownership=0)
    base.update(bad)
    cfg = azgo_hip.net_cfg(**base)
    with pytest.raises(azgo_hip.HipError) as e:
        azgo_hip.memory_need(cfg, 4, 1)
    assert e.value.code == azgo_hip.ERR_ARGUMENT


def _tensors(cfg):
    return O.init_network(cfg).tensors()


def test_upload_refuses_unknown_tensor_by_name():
    """tests/test_cuda.cpp:920-930: a tensor the pass does not know."""
    cfg = O.make_cfg(9, 1, 16, 8)
    t = dict(_tensors(cfg))
    t["block7.conv1.w"] = np.zeros(16 * 16 * 9, np.float32)
    with pytest.raises(azgo_hip.HipError) as e:
        azgo_hip.Runner(to_hip_cfg(azgo_hip, cfg), t, 4)
    assert e.value.code == azgo_hip.ERR_TENSOR and "block7.conv1.w" in str(e.value)


def test_upload_refuses_unread_tensor():
    """tests/test_cuda.cpp:934-947: a tensor of a head the config does not
    have (the ownership head's, given for a network without it) is refused,
    by name."""
    cfg = O.make_cfg(9, 1, 16, 8, ownership=1)
    t = _tensors(cfg)
    plain = to_hip_cfg(azgo_hip, O.make_cfg(9, 1, 16, 8))
    with pytest.raises(azgo_hip.HipError) as e:
        azgo_hip.Runner(plain, t, 4)
    assert e.value.code == azgo_hip.ERR_TENSOR and "ownership" in str(e.value)


def test_ownership_network_tensors():
    """With the head in the config its tensors are the network's own (the
    host-side check passes, then the runner needs a GPU); without them the
    first missing one is named."""
    cfg = O.make_cfg(9, 1, 16, 8, ownership=1)
    hcfg = to_hip_cfg(azgo_hip, cfg)
    if not azgo_hip.available()[0]:
        with pytest.raises(azgo_hip.HipError) as e:
            azgo_hip.Runner(hcfg, _tensors(cfg), 4)
        assert e.value.code == azgo_hip.ERR_UNAVAILABLE
    t = dict(_tensors(cfg))
    del t["ownership.bn.runVar"]
    with pytest.raises(azgo_hip.HipError) as e:
        azgo_hip.Runner(hcfg, t, 4)
    assert e.value.code == azgo_hip.ERR_TENSOR and "ownership.bn.runVar" in str(e.value)
    # The slot's extra [B][A] ownership buffer.
    plain = to_hip_cfg(azgo_hip, O.make_cfg(9, 1, 16, 8))
    al = lambda f: (f + 63) // 64 * 64   # noqa: E731
    d_slot = (azgo_hip.memory_need(hcfg, 64, 2) - azgo_hip.memory_need(hcfg, 64, 1)) - \
             (azgo_hip.memory_need(plain, 64, 2) - azgo_hip.memory_need(plain, 64, 1))
    assert d_slot == 4 * al(64 * 81)


def test_upload_refuses_missing_and_wrong_size():
    cfg = O.make_cfg(9, 1, 16, 8)
    t = dict(_tensors(cfg))
    del t["value.fc1.b"]
    with pytest.raises(azgo_hip.HipError) as e:
        azgo_hip.Runner(to_hip_cfg(azgo_hip, cfg), t, 4)
    assert e.value.code == azgo_hip.ERR_TENSOR and "value.fc1.b" in str(e.value)
    t = dict(_tensors(cfg))
    t["policy.fc.b"] = t["policy.fc.b"][:-1]
    with pytest.raises(azgo_hip.HipError) as e:
        azgo_hip.Runner(to_hip_cfg(azgo_hip, cfg), t, 4)
    assert e.value.code == azgo_hip.ERR_TENSOR and "policy.fc.b" in str(e.value)


def test_runner_argument_checks():
    cfg = O.make_cfg(9, 1, 16, 8)
    t = _tensors(cfg)
    for mb, slots in ((0, 1), (4, 0), (4, 3)):
        with pytest.raises(azgo_hip.HipError) as e:
            azgo_hip.Runner(to_hip_cfg(azgo_hip, cfg), t, mb, slots)
        assert e.value.code == azgo_hip.ERR_ARGUMENT


def test_memory_groups_refused_before_any_device_work():
    """No group, or a group with a count below 1, is an argument error
    (checkCudaInferenceMemory's "no hubs" / "bad arguments"), found on the host."""
    cfg = to_hip_cfg(azgo_hip, O.WORKLOADS[1].cfg)
    for groups in ([], [(1, 2, 0)], [(0, 2, 8)], [(1, 0, 8)], [(1, 2, 8), (1, 1, -1)]):
        with pytest.raises(azgo_hip.HipError) as e:
            azgo_hip.check_memory_groups(cfg, groups)
        assert e.value.code == azgo_hip.ERR_ARGUMENT, groups
        assert "checkHipInferenceMemory" in str(e.value)


def test_hooks_round_trip():
    azgo_hip.set_hub_chaos_seed(12345)
    assert azgo_hip.hub_chaos_seed() == 12345
    azgo_hip.set_hub_chaos_seed(0)
    assert azgo_hip.hub_chaos_seed() == 0
    assert azgo_hip.passes_completed() >= 0
    azgo_hip.fail_passes_after(0)
    azgo_hip.set_copy_out_delay(0)
    azgo_hip.set_memory_limit(0)


def test_last_error_is_per_thread():
    import threading
    lib = azgo_hip.load()
    cfg = azgo_hip.net_cfg(7, 8, 1, 16, 8)
    n = C.c_size_t()
    assert lib.azh_memory_need(C.byref(cfg), 4, 1, C.byref(n)) == azgo_hip.ERR_ARGUMENT
    seen = []
    th = threading.Thread(target=lambda: seen.append(lib.azh_last_error()))
    th.start()
    th.join()
    assert seen == [b""] and b"board size 7" in lib.azh_last_error()
