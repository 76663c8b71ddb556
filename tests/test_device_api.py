"""Host-side API of the xdna device (no GPU needed): registration on import, the
torch.xdna module and the reference's public functions (xdna_train/__init__.py:3-50),
the fused-optimizer pre-hook's selection rule (device.py:408-436), parameter identity
across Module.to("xdna") (device.py:355-405)."""
from types import SimpleNamespace

import torch

import xdna_train
from xdna_train import device as dev


def test_registration_and_public_api():
    assert torch._C._get_privateuse1_backend_name() == "xdna"
    assert hasattr(torch, "xdna")
    for name in xdna_train.__all__:
        assert hasattr(xdna_train, name), name
    for name in ("is_available", "device_count", "current_device", "set_device", "synchronize",
                 "empty_cache", "memory_stats", "get_amp_supported_dtype", "manual_seed_all",
                 "device"):
        assert hasattr(torch.xdna, name), name
    assert torch.xdna.get_amp_supported_dtype() == [torch.bfloat16, torch.float32]
    assert xdna_train.wait_for_builds() is True
    assert xdna_train.autotune_result() is None
    stats = xdna_train.allocator_stats()
    assert {"cached_bytes", "fresh_allocations", "reuses"} <= set(stats)
    assert xdna_train.native_library_path().name.startswith("_C")


def test_mode_switch():
    old = xdna_train.npu_mode()
    try:
        for m in (0, 1, 2):
            xdna_train.set_npu_mode(m)
            assert xdna_train.npu_mode() == m
    finally:
        xdna_train.set_npu_mode(old)


def test_device_index_rules():
    assert dev._xdna_index(None) == 0
    assert dev._xdna_index("xdna") == 0
    assert dev._xdna_index("xdna:0") == 0
    for bad in ("xdna:1", "cpu", 3):
        try:
            dev._xdna_index(bad)
        except ValueError:
            continue
        raise AssertionError(bad)


class _FakeParam:
    def __init__(self, device_type, floating=True):
        self.device = SimpleNamespace(type=device_type)
        self._floating = floating

    def is_floating_point(self):
        return self._floating


def _fake_param(device_type, floating=True):
    return _FakeParam(device_type, floating)


def test_prefer_fused_optimizer_rule():
    p1, p2 = _fake_param("xdna"), _fake_param("xdna")
    groups = [{"params": [p1, p2], "fused": None, "foreach": None},
              {"params": [_fake_param("cpu")], "fused": None, "foreach": None},
              {"params": [_fake_param("xdna")], "fused": None, "foreach": False},
              {"params": [_fake_param("xdna", floating=False)], "fused": None, "foreach": None}]
    opt = SimpleNamespace(param_groups=groups, state={})
    dev._default_fused_step(opt, (), {})
    assert groups[0]["fused"] is True
    assert groups[1]["fused"] is None and groups[2]["fused"] is None and groups[3]["fused"] is None
    # decided once: later calls do nothing
    groups[1]["params"] = [_fake_param("xdna")]
    dev._default_fused_step(opt, (), {})
    assert groups[1]["fused"] is None


def test_module_move_keeps_parameters_only_for_xdna():
    """The move methods are wrapped once, and the swap switch is on only while a move
    targets xdna (checked without device memory: the target parser alone)."""
    for name in ("to", "to_empty", "xdna"):
        assert hasattr(getattr(torch.nn.Module, name), "__xdna_original__"), name
    assert dev._targets_xdna(dev._PARAM_MOVES["to"], ("xdna",), {})
    assert dev._targets_xdna(dev._PARAM_MOVES["to"], (torch.device("xdna:0"),), {})
    assert not dev._targets_xdna(dev._PARAM_MOVES["to"], (torch.bfloat16,), {})
    assert not dev._targets_xdna(dev._PARAM_MOVES["to"], ("cpu",), {})
    assert dev._targets_xdna(dev._PARAM_MOVES["to_empty"], (), {"device": "xdna"})
    assert not dev._targets_xdna(dev._PARAM_MOVES["to"], ("no such device",), {})
    # a CPU move leaves the switch as it was
    before = torch.__future__.get_swap_module_params_on_conversion()
    m = torch.nn.Linear(2, 2)
    m.to(torch.float64)
    assert torch.__future__.get_swap_module_params_on_conversion() == before
    assert m.weight.dtype == torch.float64


def test_wait_deadline_setting():
    old = xdna_train.device.native().wait_timeout_ms()
    try:
        xdna_train.set_wait_timeout_ms(1234)
        assert xdna_train.device.native().wait_timeout_ms() == 1234
    finally:
        xdna_train.set_wait_timeout_ms(old)
    assert xdna_train.max_wait_ms() >= 0.0
