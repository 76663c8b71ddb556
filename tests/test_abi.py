"""The C-ABI library loads, exports every function declared in include/xdna_hip.h, and
handles its failure paths on the host (no device work is issued by these tests).

Failure handling follows the reference shim (xrt_shim.cpp:139-233): an error returns
-1 with a thread-local message; a poisoned process refuses launches and leaks frees.
"""
import re
from pathlib import Path

import numpy as np
import pytest

from xdna_train import hip_abi

HEADER = Path(__file__).resolve().parents[1] / "include" / "xdna_hip.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(xdna_\w+)\s*\(", text))


def test_every_declared_symbol_is_exported_and_bound():
    lib = hip_abi.load()
    names = _declared()
    assert len(names) >= 30
    for n in names:
        assert hasattr(lib, n), f"{n} not exported by {hip_abi.LIB_PATH.name}"
    assert names == set(hip_abi.SIGNATURES), "hip_abi.SIGNATURES out of sync with the header"


def test_invalid_arguments_report_errors():
    lib = hip_abi.load()
    rc = lib.xdna_conv3x3w_pack_input_strips_range_bf16(None, None, -1, 1, 1, 1, 1, 1, 0, 1, 0, 1, None)
    assert rc == -1 and "invalid geometry" in hip_abi.last_error()
    rc = lib.xdna_conv3x3w_unpack_output_bf16(None, None, 1, 1, 1, 200, 200, 0, None)
    assert rc == -1 and "invalid geometry" in hip_abi.last_error()
    rc = lib.xdna_gemm_bf16(None, None, None, None, 1, 1, 1, 1, 0, 0, 0, 0, 0, 0, 0, 0, 0, 1, 0, 0,
                            1.0, 0.0, None)
    assert rc == -1 and "invalid" in hip_abi.last_error()
    assert lib.xdna_conv3x3_fwd_workspace_bytes(0, 1, 1, 1, 1) == 0
    # zero-sized work is a successful no-op
    assert lib.xdna_conv3x3w_pack_input_bf16(None, None, 0, 3, 4, 4, 1, None) == 0


def test_geometry_matches_reference_plan():
    lib = hip_abi.load()
    out = (hip_abi.L * 7)()
    # C1: [16,128,36,36] -> S=1, wp=38, groups 12, chunks 2 (torch_xdna_device.cpp:2112-2157)
    assert lib.xdna_conv3x3w_geometry(16, 128, 36, 36, out) == 0
    assert list(out) == [1, 36, 36, 38, 12, 2, 16 * 38 * 38]
    # C2 max: N64 C512 H72 -> S=3, So=24, wp=28, groups 195, chunks 8
    assert lib.xdna_conv3x3w_geometry(64, 512, 72, 72, out) == 0
    assert list(out)[:6] == [3, 24, 26, 28, 195, 8]


def test_injected_failure_and_poisoning():
    lib = hip_abi.load()
    lib.xdna_hip_reset_failure_state()
    try:
        # the next launch fails before touching the device
        assert lib.xdna_hip_inject_failure(1, 0) == 0
        rc = lib.xdna_conv3x3w_pack_input_bf16(None, None, 1, 1, 1, 1, 1, None)
        assert rc == -1 and "injected failure" in hip_abi.last_error()
        assert lib.xdna_hip_poisoned() == 0
        # a poisoning failure: every later launch is refused and frees leak
        assert lib.xdna_hip_inject_failure(1, 1) == 0
        assert lib.xdna_conv3x3w_pack_input_bf16(None, None, 1, 1, 1, 1, 1, None) == -1
        assert lib.xdna_hip_poisoned() == 1
        assert lib.xdna_conv3x3w_pack_input_bf16(None, None, 1, 1, 1, 1, 1, None) == -1
        assert "poisoned" in hip_abi.last_error()
        assert lib.xdna_hip_free(hip_abi.P(0x1000)) == 0  # leaked, not handed to the driver
    finally:
        lib.xdna_hip_reset_failure_state()
    assert lib.xdna_hip_poisoned() == 0


def test_injected_wait_timeout_is_distinct_and_poisons():
    """The dispatch deadline (xrt_shim.cpp:57-90, 174-233): a wait past it returns -2, not
    the error status -1, names what it waited for, and poisons the process.  Forced from
    the host by the injection hook: the injected wait never touches the device."""
    lib = hip_abi.load()
    lib.xdna_hip_reset_failure_state()
    cases = [(lambda: lib.xdna_hip_stream_synchronize(None), "the stream"),
             (lambda: lib.xdna_hip_device_synchronize(), "the device"),
             (lambda: lib.xdna_hip_event_synchronize(None), "an event")]
    try:
        for wait, what in cases:
            assert lib.xdna_hip_inject_wait_timeout(1) == 0
            assert wait() == -2
            msg = hip_abi.last_error()
            assert msg.startswith("deadline:") and what in msg and "poisoned" in msg
            assert lib.xdna_hip_poisoned() == 1
            # poisoned: launches are refused, frees leak
            assert lib.xdna_conv3x3w_pack_input_bf16(None, None, 1, 1, 1, 1, 1, None) == -1
            assert "poisoned" in hip_abi.last_error()
            lib.xdna_hip_reset_failure_state()
        # the n-th wait from now, not the next one: a 0 disables it again
        assert lib.xdna_hip_inject_wait_timeout(0) == 0
        assert lib.xdna_hip_inject_wait_timeout(-1) == -1
    finally:
        lib.xdna_hip_reset_failure_state()
    assert lib.xdna_hip_poisoned() == 0


def test_wait_deadline_setting_and_real_waits_are_not_timeouts():
    lib = hip_abi.load()
    old = lib.xdna_hip_wait_timeout_ms()
    try:
        assert lib.xdna_hip_set_wait_timeout_ms(250) == 0
        assert lib.xdna_hip_wait_timeout_ms() == 250
        assert lib.xdna_hip_set_wait_timeout_ms(-5) == -1
    finally:
        lib.xdna_hip_set_wait_timeout_ms(old)
    # without injection a wait either completes (GPU present) or fails as an error (no
    # device here): never a timeout
    lib.xdna_hip_reset_failure_state()
    try:
        assert lib.xdna_hip_stream_synchronize(None) in (0, -1)
    finally:
        lib.xdna_hip_reset_failure_state()


def test_error_message_is_thread_local():
    import threading

    lib = hip_abi.load()
    lib.xdna_conv3x3w_pack_input_bf16(None, None, -1, 1, 1, 1, 1, None)
    seen = {}

    def other():
        seen["msg"] = hip_abi.last_error()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == ""
    assert "invalid geometry" in hip_abi.last_error()
