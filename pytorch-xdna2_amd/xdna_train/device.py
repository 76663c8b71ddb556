"""Registration of the ``xdna`` PrivateUse1 device on MI355X and its Python API.

Mirrors the reference's ``xdna_train/device.py``: the same public functions
(``__init__.py:3-50``), the ``torch.xdna`` device module (``device.py:53-97``), the
rename of PrivateUse1 (``:245-252``), autograd on the calling thread (``:254-261``),
parameter identity across ``Module.to("xdna")`` (``:355-405``) and the fused-optimizer
hooks (``:408-452``).  What the reference spends on its NPU toolchain (IRON builds,
build waiting, the step autotuner across NPU modes, XRT coherency) has no counterpart
here: kernels are compiled ahead of time for gfx950 and HBM is coherent for the stream;
those functions keep their names and answer trivially.
"""
from __future__ import annotations

import ctypes
import os
import sys
from pathlib import Path
from types import SimpleNamespace

import torch

_ROOT = Path(__file__).resolve().parent
_INITIALIZED = False
_C = None

LIB_PATH = _ROOT / "_lib" / "libxdna_hip.so"


def _device_index(device=None, optional: bool = False) -> int:
    del optional
    if device is None:
        return 0
    if isinstance(device, int):
        index = device
    else:
        d = torch.device(device)
        if d.type != "xdna":
            raise ValueError(f"expected xdna device, got {d}")
        index = 0 if d.index is None else d.index
    if index != 0:
        raise ValueError("only xdna:0 is supported (one MI355X per process)")
    return index


class _DeviceContext:
    """``with torch.xdna.device(i):`` (torch.load and similar code enter it)."""

    def __init__(self, device):
        self.index = _device_index(device)
        self.prev = 0

    def __enter__(self):
        self.prev = int(_C.current_device())
        _C.set_device(self.index)
        return self

    def __exit__(self, *exc):
        _C.set_device(self.prev)
        return False


class _XdnaDeviceModule:
    _utils = SimpleNamespace(_get_device_index=_device_index)
    device = _DeviceContext

    @staticmethod
    def is_available() -> bool:
        return bool(_C.is_available())

    @staticmethod
    def device_count() -> int:
        return int(_C.device_count())

    @staticmethod
    def current_device() -> int:
        return int(_C.current_device())

    @staticmethod
    def set_device(device) -> None:
        _C.set_device(_device_index(device))

    @staticmethod
    def synchronize(device=None) -> None:
        if device is not None:
            _device_index(device)
        _C.synchronize()

    @staticmethod
    def empty_cache() -> None:
        _C.empty_cache()

    @staticmethod
    def memory_stats() -> dict[str, int]:
        return dict(_C.allocator_stats())

    @staticmethod
    def get_amp_supported_dtype():
        return [torch.bfloat16, torch.float32]

    @staticmethod
    def _is_in_bad_fork() -> bool:
        return False

    @staticmethod
    def is_initialized() -> bool:
        return _INITIALIZED

    @staticmethod
    def manual_seed(seed: int) -> None:
        torch.random.default_generator.manual_seed(seed)

    @staticmethod
    def manual_seed_all(seed: int) -> None:
        torch.random.default_generator.manual_seed(seed)


def _load_native():
    """Loads libxdna_hip.so (the C ABI) and the _C extension built next to it.  Raises
    ImportError when either is missing: there is no CPU substitute for the kernels."""
    global _C
    if _C is not None:
        return _C
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is missing: run `python pytorch-xdna2_amd/build_native.py`")
    ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
    from . import _C as native  # noqa: PLC0415

    _C = native
    return _C


def register_xdna_device() -> None:
    global _INITIALIZED
    if _INITIALIZED:
        return
    _load_native()
    # PyTorch-ROCm initializes its caching allocator lazily from Python; kernels the
    # fallback reaches from C++ need it ready.
    if _C.is_available() and torch.cuda.is_available():
        torch.cuda.init()
    current = torch._C._get_privateuse1_backend_name()
    if current == "privateuseone":
        torch.utils.rename_privateuse1_backend("xdna")
    elif current != "xdna":
        raise RuntimeError(
            f"PrivateUse1 is already claimed by backend {current!r}; "
            "xdna cannot coexist with another PrivateUse1 backend in one process.")

    # Backward on the calling thread, as for CPU tensors (the reference's reason:
    # device-thread hand-off cost; here also one stream, one thread).
    if os.environ.get("XDNA_AUTOGRAD_THREAD", "0") != "1":
        torch.autograd.set_multithreading_enabled(False)

    if not hasattr(torch, "xdna"):
        torch._register_device_module("xdna", _XdnaDeviceModule)
    torch.utils.generate_methods_for_privateuse1_backend(
        for_tensor=True, for_module=True, for_storage=False)
    try:
        torch.set_autocast_dtype("xdna", torch.bfloat16)
    except (RuntimeError, AttributeError):
        pass
    _install_scoped_param_swap()

    mode = os.environ.get("XDNA_NPU_MODE")
    if mode is not None:
        _C.set_npu_mode(int(mode))

    from torch.optim.optimizer import (
        register_optimizer_step_post_hook,
        register_optimizer_step_pre_hook,
    )

    register_optimizer_step_post_hook(_bump_fused_param_versions)
    if os.environ.get("XDNA_FUSED_OPTIMIZER", "1") == "1":
        register_optimizer_step_pre_hook(_prefer_fused_optimizer)
    _INITIALIZED = True


class _SwapModuleParams:
    """Use torch.utils.swap_tensors while a module moves to xdna.

    PyTorch keeps Parameter identity in Module.to() only for backends it treats as
    shallow-copy compatible, not for PrivateUse1: without swapping, model.to("xdna")
    would create new Parameter objects and an optimizer built before the move would
    keep updating the old CPU tensors.  Enabled only for conversions to xdna.
    """

    def __enter__(self):
        self.prev = torch.__future__.get_swap_module_params_on_conversion()
        torch.__future__.set_swap_module_params_on_conversion(True)

    def __exit__(self, *exc):
        torch.__future__.set_swap_module_params_on_conversion(self.prev)


def _install_scoped_param_swap() -> None:
    import functools

    module = torch.nn.Module
    if getattr(module.to, "_xdna_scoped_swap", False):
        return

    def is_xdna(device) -> bool:
        return device is not None and torch.device(device).type == "xdna"

    def scoped(fn, targets_xdna):
        @functools.wraps(fn)
        def wrapper(self, *args, **kwargs):
            if not targets_xdna(*args, **kwargs):
                return fn(self, *args, **kwargs)
            with _SwapModuleParams():
                return fn(self, *args, **kwargs)

        wrapper._xdna_scoped_swap = True
        return wrapper

    def to_targets(*args, **kwargs):
        try:
            device = torch._C._nn._parse_to(*args, **kwargs)[0]
        except Exception:
            return False  # Module.to raises its own error
        return is_xdna(device)

    module.to = scoped(module.to, to_targets)
    module.to_empty = scoped(module.to_empty, lambda *, device=None, **k: is_xdna(device))
    if hasattr(module, "xdna"):
        module.xdna = scoped(module.xdna, lambda *a, **k: True)


def _prefer_fused_optimizer(optimizer, args, kwargs) -> None:
    """Default xdna optimizers to the fused kernel (one HIP launch per step and dtype
    instead of ~10 foreach launches).  Only param groups that left both ``fused`` and
    ``foreach`` unset, hold only xdna floating-point parameters and have no state yet are
    changed, so it happens before the first step or not at all.
    XDNA_FUSED_OPTIMIZER=0 disables it."""
    if getattr(optimizer, "_xdna_fused_checked", False):
        return
    optimizer._xdna_fused_checked = True
    for group in optimizer.param_groups:
        if ("fused" not in group or group.get("fused") is not None
                or group.get("foreach") is not None or group.get("differentiable")):
            continue
        params = group["params"]
        if params and all(p.device.type == "xdna" and p.is_floating_point()
                          and not optimizer.state.get(p) for p in params):
            group["fused"] = True


def _bump_fused_param_versions(optimizer, args, kwargs) -> None:
    """Marks parameters written by a fused optimizer step as modified (version counters
    are what caches of prepared weights key on)."""
    for group in optimizer.param_groups:
        if not group.get("fused"):
            continue
        params = [p for p in group["params"] if p.device.type == "xdna"]
        if params:
            torch.autograd.graph.increment_version(params)


def try_register_xdna_device() -> bool:
    """Registers the device if possible (called on import); on failure warns with the
    cause instead of failing later with "No module named 'torch.xdna'"."""
    try:
        register_xdna_device()
    except (ImportError, RuntimeError, OSError) as e:
        import warnings

        warnings.warn(f"xdna_train: xdna device not registered: {type(e).__name__}: {e}",
                      RuntimeWarning, stacklevel=2)
        return False
    return True


def is_available() -> bool:
    try:
        register_xdna_device()
    except (ImportError, RuntimeError, OSError):
        return False
    return _XdnaDeviceModule.is_available()


def synchronize(device=None) -> None:
    """Waits for all queued device work, weight gradients included (the reference's
    synchronize leaves deferred NPU weight gradients pending, README.md:117-118)."""
    register_xdna_device()
    _XdnaDeviceModule.synchronize(device)


def empty_cache() -> None:
    register_xdna_device()
    _C.empty_cache()


def allocator_stats() -> dict[str, int]:
    register_xdna_device()
    return dict(_C.allocator_stats())


def async_dw_stats() -> dict:
    """Weight-gradient launches: "jobs" counts HIP weight gradients; they are ordered
    on the stream before any reader, so there is nothing to kick or learn."""
    register_xdna_device()
    return dict(_C.async_dw_stats())


def autotune_result() -> dict | None:
    """Always None: there are no slower-than-CPU device paths to tune away."""
    return None


def set_npu_mode(mode: int) -> None:
    """2: all HIP paths, 1: no HIP weight gradient, 0: every op through the generic
    PyTorch-ROCm fallback (same switch as the reference's NPU modes)."""
    register_xdna_device()
    _C.set_npu_mode(int(mode))


def npu_mode() -> int:
    register_xdna_device()
    return int(_C.npu_mode())


def set_general_conv_mode(mode: int) -> None:
    """Convolutions outside the 3x3 / stride-1 path (strided, 1x1, 9x9, ...): 0 on
    PyTorch-ROCm (MIOpen), 1 (default) on the general HIP kernels where those measured
    faster, 2 on the general HIP kernels always.  XDNA_GENERAL_CONV sets the initial value.
    No reference counterpart (the reference runs these on its CPU)."""
    register_xdna_device()
    _C.set_general_conv_mode(int(mode))


def general_conv_mode() -> int:
    register_xdna_device()
    return int(_C.general_conv_mode())


def set_wgrad_form(form: int) -> None:
    """Weight gradient of the 3x3 / stride-1 convs: 0 (default) and 2 the packed-rows
    form (dY read in the packed form its input gradient used, x in the packed form its
    forward used), 1 the channel-major form (x and dY copied channel-major).  Both sum in
    fp32 and round once to bf16, in different orders.  Images wider than 142 always take
    the rows form.  XDNA_WGRAD_FORM sets the initial value.  No reference counterpart."""
    register_xdna_device()
    _C.set_wgrad_form(int(form))


def wgrad_form() -> int:
    register_xdna_device()
    return int(_C.wgrad_form())


def set_conv_layout(layout: int) -> None:
    """Row layout of the packed operands of the 3x3 convs: 1 (default) tight strips
    (images wider than 36 as strips of up to 36 columns without zero columns), 0 the
    reference's conv3x3w layout (strips of up to 34 columns between zero columns).  The
    results agree to the conv tolerance (the sums run in other orders).  XDNA_CONV_LAYOUT
    sets the initial value.  No reference counterpart."""
    register_xdna_device()
    _C.set_conv_layout(int(layout))


def conv_layout() -> int:
    register_xdna_device()
    return int(_C.conv_layout())


def wait_for_builds(timeout: float | None = None) -> bool:
    """Kernels are compiled ahead of time: nothing is ever pending."""
    del timeout
    register_xdna_device()
    return True


def reset_mapped_cpu_stats() -> None:
    register_xdna_device()
    _C.reset_mapped_cpu_stats()


def mapped_cpu_stats() -> dict[str, dict[str, float | int]]:
    """Per-path counters (calls, host ms): ``hip_conv3x3.{fwd,dx,dw}.run``,
    ``hip_gemm.*``, ``hip_adam.run`` and the ``*.rocm`` fallbacks of the hot ops."""
    register_xdna_device()
    return {str(k): dict(v) for k, v in dict(_C.mapped_cpu_stats()).items()}


def reset_fallback_stats() -> None:
    register_xdna_device()
    _C.reset_fallback_stats()


def fallback_stats() -> dict[str, dict[str, float | int]]:
    """Operators served by the generic fallback (calls; host ms with
    XDNA_PROFILE_FALLBACK=1)."""
    register_xdna_device()
    return {str(k): dict(v) for k, v in dict(_C.fallback_stats()).items()}


def native_library_path() -> Path:
    register_xdna_device()
    return Path(_C.__file__).resolve()


def is_xrt_backed(tensor: torch.Tensor) -> bool:
    """False: xdna tensors live in HIP device memory, not XRT buffer objects."""
    del tensor
    return False


def bo_handle(tensor: torch.Tensor) -> int:
    """The device address of the tensor's data (the nearest thing to a BO handle)."""
    register_xdna_device()
    return int(_C.data_ptr(tensor))


def coherency_state(tensor: torch.Tensor) -> int:
    """0 (Clean): device memory is coherent for the stream; there is no host copy."""
    del tensor
    return 0


def cpu_mm(lhs: torch.Tensor, rhs: torch.Tensor) -> torch.Tensor:
    """The reference's CPU matmul on device tensors; here the plain product on host copies."""
    return (lhs.cpu() @ rhs.cpu()).to(lhs.device)
