"""The ``xdna`` device on one MI355X: registration and the Python API.

Public names follow the reference package (``xdna_train/__init__.py:3-50``, the
``torch.xdna`` module of ``device.py:53-97``) so unchanged scripts keep working.  The
design here is its own:

* one ``_Backend`` object owns the native pieces (``_lib/libxdna_hip.so``, the C ABI of
  the gfx950 kernels, and the ``_C`` extension that registers PrivateUse1 over it) and
  registers the device once; every API function goes through it;
* ``torch.xdna`` is a plain namespace module built from functions;
* two behaviours the reference documents are kept as rules:
  - moving a module *to* xdna keeps its Parameter objects (``device.py:355-405``): the
    module-moving methods named in ``_PARAM_MOVES`` run with PyTorch's swap-on-conversion
    switched on when their target device is xdna;
  - optimizers default to their fused kernel on xdna (``device.py:408-436``): a group that
    left ``fused`` and ``foreach`` unset, holding only fresh xdna floating-point
    parameters, is switched to ``fused=True`` before its first step.

The reference's version bump after fused steps (``device.py:439-452``) has no counterpart:
the backend keeps a write epoch per allocation that the fused kernels (and every other
xdna write) advance, and its caches key on that.  What the reference spends on its NPU
toolchain (IRON builds, the step autotuner, XRT coherency) has nothing to do here:
kernels are compiled ahead of time for gfx950 and HBM is coherent on the stream, so those
functions keep their names and answer with constants.
"""
from __future__ import annotations

import contextlib
import ctypes
import functools
import os
import types
from pathlib import Path

import torch

_PKG = Path(__file__).resolve().parent
_HIP_LIBRARY = _PKG / "_lib" / "libxdna_hip.so"
_NAME = "xdna"


class _Backend:
    """Loads the native libraries on first use and registers the device once."""

    def __init__(self):
        self.ext = None
        self.registered = False

    def native(self):
        if self.ext is None:
            if not _HIP_LIBRARY.is_file():
                raise ImportError(f"{_HIP_LIBRARY} is missing: build it with "
                                  "`python pytorch-xdna2_amd/build_native.py`")
            # the extension resolves the C ABI's symbols from this global load
            ctypes.CDLL(str(_HIP_LIBRARY), mode=ctypes.RTLD_GLOBAL)
            from . import _C  # noqa: PLC0415

            self.ext = _C
        return self.ext

    def register(self):
        if self.registered:
            return self.ext
        ext = self.native()
        claimed = torch._C._get_privateuse1_backend_name()
        if claimed not in ("privateuseone", _NAME):
            raise RuntimeError(f"PrivateUse1 already belongs to {claimed!r}; "
                               "the xdna backend cannot share a process with it")
        if ext.is_available() and torch.cuda.is_available():
            # the fallback reaches PyTorch-ROCm kernels from C++: its allocator must exist
            torch.cuda.init()
        if claimed != _NAME:
            torch.utils.rename_privateuse1_backend(_NAME)
        if os.environ.get("XDNA_AUTOGRAD_THREAD", "0") != "1":
            # backward runs on the calling thread, as for CPU tensors: one stream, no
            # device-thread hand-off (the reference's choice, device.py:254-261)
            torch.autograd.set_multithreading_enabled(False)
        if not hasattr(torch, _NAME):
            torch._register_device_module(_NAME, _device_module)
        torch.utils.generate_methods_for_privateuse1_backend(
            for_tensor=True, for_module=True, for_storage=False)
        with contextlib.suppress(RuntimeError, AttributeError):
            torch.set_autocast_dtype(_NAME, torch.bfloat16)
        _keep_parameters_on_move()
        if (mode := os.environ.get("XDNA_NPU_MODE")) is not None:
            ext.set_npu_mode(int(mode))
        if os.environ.get("XDNA_FUSED_OPTIMIZER", "1") == "1":
            from torch.optim.optimizer import register_optimizer_step_pre_hook

            register_optimizer_step_pre_hook(_default_fused_step)
        self.registered = True
        return ext


_backend = _Backend()


def native():
    """The registered ``_C`` extension (registers the device on first use)."""
    return _backend.register()


def _api(fn):
    """Public functions make sure the device is registered before they run."""

    @functools.wraps(fn)
    def call(*args, **kwargs):
        _backend.register()
        return fn(*args, **kwargs)

    return call


# ---------------------------------------------------------------------------------------
# torch.xdna
# ---------------------------------------------------------------------------------------
def _xdna_index(device=None, optional: bool = False) -> int:
    """Index named by an xdna device spec (None, int, str or torch.device).  One GPU per
    process: xdna:0 is the only device."""
    del optional
    if device is None:
        return 0
    spec = torch.device(_NAME, device) if isinstance(device, int) else torch.device(device)
    if spec.type != _NAME:
        raise ValueError(f"not an xdna device: {spec}")
    if spec.index not in (None, 0):
        raise ValueError("xdna:0 is the only device (one MI355X per process)")
    return 0


@contextlib.contextmanager
def _device_scope(device):
    """``with torch.xdna.device(d):`` (torch.load and friends enter it)."""
    index = _xdna_index(device)
    ext = native()
    before = int(ext.current_device())
    ext.set_device(index)
    try:
        yield index
    finally:
        ext.set_device(before)


def _synchronize_device(device=None) -> None:
    _xdna_index(device)
    native().synchronize()


def _seed(seed: int) -> None:
    # the device has no generator of its own: random ops draw from the CPU generator
    torch.random.default_generator.manual_seed(int(seed))


_device_module = types.ModuleType("torch.xdna", "The xdna device (one MI355X, HIP memory).")
_device_module.__dict__.update(
    _utils=types.SimpleNamespace(_get_device_index=_xdna_index),
    device=_device_scope,
    is_available=lambda: bool(native().is_available()),
    device_count=lambda: int(native().device_count()),
    current_device=lambda: int(native().current_device()),
    set_device=lambda device: native().set_device(_xdna_index(device)),
    synchronize=_synchronize_device,
    empty_cache=lambda: native().empty_cache(),
    memory_stats=lambda: dict(native().allocator_stats()),
    get_amp_supported_dtype=lambda: [torch.bfloat16, torch.float32],
    is_initialized=lambda: _backend.registered,
    _is_in_bad_fork=lambda: False,
    manual_seed=_seed,
    manual_seed_all=_seed,
)


# ---------------------------------------------------------------------------------------
# Rule 1: Module.to("xdna") and friends keep the Parameter objects
# ---------------------------------------------------------------------------------------
# PyTorch keeps Parameter identity across a device move only for backends it treats as
# shallow-copy compatible, which PrivateUse1 is not: without swapping, model.to("xdna")
# would make new Parameters and an optimizer built earlier would keep the CPU ones.
# Method name -> its target device from the call's arguments.
_PARAM_MOVES = {
    "to": lambda *a, **k: torch._C._nn._parse_to(*a, **k)[0],
    "to_empty": lambda *a, device=None, **k: device,
    _NAME: lambda *a, **k: _NAME,
}


def _targets_xdna(target_of, args, kwargs) -> bool:
    try:
        target = target_of(*args, **kwargs)
    except Exception:  # malformed call: the method itself reports it
        return False
    return target is not None and torch.device(target).type == _NAME


def _swap_on_xdna_move(method, target_of):
    @functools.wraps(method)
    def move(module, *args, **kwargs):
        if not _targets_xdna(target_of, args, kwargs):
            return method(module, *args, **kwargs)
        future = torch.__future__
        before = future.get_swap_module_params_on_conversion()
        future.set_swap_module_params_on_conversion(True)
        try:
            return method(module, *args, **kwargs)
        finally:
            future.set_swap_module_params_on_conversion(before)

    move.__xdna_original__ = method
    return move


def _keep_parameters_on_move() -> None:
    for name, target_of in _PARAM_MOVES.items():
        method = getattr(torch.nn.Module, name, None)
        if method is not None and not hasattr(method, "__xdna_original__"):
            setattr(torch.nn.Module, name, _swap_on_xdna_move(method, target_of))


# ---------------------------------------------------------------------------------------
# Rule 2: fused optimizer steps by default
# ---------------------------------------------------------------------------------------
def _implementation_unset(group: dict) -> bool:
    """The group supports ``fused`` and the user chose neither fused nor foreach."""
    return ("fused" in group and group["fused"] is None and group.get("foreach") is None
            and not group.get("differentiable"))


def _fresh_xdna_floats(optimizer, params) -> bool:
    return bool(params) and all(
        p.device.type == _NAME and p.is_floating_point() and not optimizer.state.get(p)
        for p in params)


def _default_fused_step(optimizer, args, kwargs) -> None:
    """Optimizer pre-step hook: one fused HIP launch per step and dtype instead of ~10
    foreach launches.  Decided once per optimizer, before its first step.
    XDNA_FUSED_OPTIMIZER=0 disables it."""
    del args, kwargs
    if vars(optimizer).get("_xdna_fused_decided"):
        return
    optimizer._xdna_fused_decided = True
    for group in optimizer.param_groups:
        if _implementation_unset(group) and _fresh_xdna_floats(optimizer, group["params"]):
            group["fused"] = True


# ---------------------------------------------------------------------------------------
# Public functions (names of the reference's xdna_train/__init__.py)
# ---------------------------------------------------------------------------------------
def register_xdna_device() -> None:
    _backend.register()


def try_register_xdna_device() -> bool:
    """Registers on import; on failure warns with the cause (else the first sign would
    be a confusing "No module named 'torch.xdna'" much later)."""
    try:
        _backend.register()
    except (ImportError, RuntimeError, OSError) as err:
        import warnings

        warnings.warn(f"xdna_train: xdna device not registered: {type(err).__name__}: {err}",
                      RuntimeWarning, stacklevel=2)
        return False
    return True


def is_available() -> bool:
    try:
        return bool(_backend.register().is_available())
    except (ImportError, RuntimeError, OSError):
        return False


@_api
def synchronize(device=None) -> None:
    """Waits for all queued device work, weight gradients included (the reference leaves
    deferred NPU weight gradients pending here, README.md:117-118).  Bounded by the
    dispatch deadline (``set_wait_timeout_ms``)."""
    _device_module.synchronize(device)


@_api
def empty_cache() -> None:
    native().empty_cache()


@_api
def allocator_stats() -> dict[str, int]:
    return dict(native().allocator_stats())


@_api
def async_dw_stats() -> dict:
    """"jobs" counts HIP weight gradients.  They are stream-ordered before every reader,
    so there is no helper thread to kick and nothing to learn (both stay 0)."""
    return dict(native().async_dw_stats())


def autotune_result() -> dict | None:
    """None: no device path is slower than the CPU, so there is nothing to tune away."""
    return None


@_api
def set_npu_mode(mode: int) -> None:
    """2 every HIP path, 1 no HIP weight gradient, 0 every op through the generic
    PyTorch-ROCm fallback (the reference's NPU modes)."""
    native().set_npu_mode(int(mode))


@_api
def npu_mode() -> int:
    return int(native().npu_mode())


@_api
def set_general_conv_mode(mode: int) -> None:
    """Convolutions outside the 3x3 and 1x1 paths (strided, 5x5, 9x9, ...): 0 PyTorch-ROCm
    (MIOpen), 1 the general HIP kernels where they measured faster than MIOpen, 2 (default)
    the general HIP kernels always (MIOpen misses the conv bar on some layers).
    XDNA_GENERAL_CONV sets the initial value.  No reference counterpart (the reference runs
    these on its CPU)."""
    native().set_general_conv_mode(int(mode))


@_api
def general_conv_mode() -> int:
    return int(native().general_conv_mode())


@_api
def set_wgrad_form(form: int) -> None:
    """3x3 weight gradient: 0 (default) and 2 the packed-rows form (x and dY in the packed
    forms their forward and input gradient used), 1 the channel-major form.  Both sum in
    fp32 and round once.  Images wider than 142 always take the rows form.
    XDNA_WGRAD_FORM sets the initial value.  No reference counterpart."""
    native().set_wgrad_form(int(form))


@_api
def wgrad_form() -> int:
    return int(native().wgrad_form())


@_api
def set_conv_layout(layout: int) -> None:
    """Row layout of the 3x3 conv operands: 1 (default) tight strips of up to 36 columns
    without zero columns, 0 the reference's conv3x3w layout.  Results agree to the conv
    tolerance.  XDNA_CONV_LAYOUT sets the initial value.  No reference counterpart."""
    native().set_conv_layout(int(layout))


@_api
def conv_layout() -> int:
    return int(native().conv_layout())


@_api
def set_bfp16_emulation(on: bool) -> None:
    """Emulate the reference NPU's conv arithmetic on the 3x3 / stride-1 forward and
    input-gradient convs: activations and weights quantized to BFP16 (bfp16ebs8 blocks of
    8 channels), the running sum stored as bf16 after every 64-channel chunk and tap, the
    bias added after (benchmarks/bfp16_training_gate.py:1-20 restates it; kernel
    _designs/conv3x3w_kernel.cc).  Weight gradients stay exact.  Off by default: the
    default arithmetic is the reference's CPU bf16 path.  XDNA_BFP16_EMULATION=1 sets it
    at start-up."""
    native().set_bfp16_emulation(bool(on))


@_api
def bfp16_emulation() -> bool:
    return bool(native().bfp16_emulation())


@_api
def set_wait_timeout_ms(ms: int) -> None:
    """Deadline of every host wait on the device (default 30000, XDNA_WAIT_TIMEOUT_MS;
    0 = none).  A wait past it raises and poisons the process (xrt_shim.cpp:57-90)."""
    native().set_wait_timeout_ms(int(ms))


@_api
def max_wait_ms() -> float:
    """Longest completed host wait so far, in ms (to size the deadline)."""
    return float(native().max_wait_ms())


@_api
def wait_for_builds(timeout: float | None = None) -> bool:
    """Kernels are compiled ahead of time: nothing is ever pending."""
    del timeout
    return True


@_api
def reset_mapped_cpu_stats() -> None:
    native().reset_mapped_cpu_stats()


@_api
def mapped_cpu_stats() -> dict[str, dict[str, float | int]]:
    """Per-path counters (calls, host ms): ``hip_conv3x3.{fwd,dx,dw}.run``, ``hip_gemm.*``,
    ``hip_adam.run`` and the ``*.rocm`` fallbacks of the hot ops."""
    return {str(k): dict(v) for k, v in dict(native().mapped_cpu_stats()).items()}


@_api
def reset_fallback_stats() -> None:
    native().reset_fallback_stats()


@_api
def fallback_stats() -> dict[str, dict[str, float | int]]:
    """Operators served by the generic fallback (calls; host ms with
    XDNA_PROFILE_FALLBACK=1)."""
    return {str(k): dict(v) for k, v in dict(native().fallback_stats()).items()}


@_api
def native_library_path() -> Path:
    return Path(native().__file__).resolve()


def is_xrt_backed(tensor: torch.Tensor) -> bool:
    """False: xdna tensors live in HIP device memory, never in XRT buffer objects."""
    del tensor
    return False


@_api
def bo_handle(tensor: torch.Tensor) -> int:
    """Device address of the tensor's data, the closest thing to a BO handle here."""
    return int(native().data_ptr(tensor))


def coherency_state(tensor: torch.Tensor) -> int:
    """0 (clean): HBM is coherent on the stream and there is no host copy to track."""
    del tensor
    return 0


def cpu_mm(lhs: torch.Tensor, rhs: torch.Tensor) -> torch.Tensor:
    """The reference's CPU matmul of device tensors: the product of host copies."""
    return (lhs.cpu() @ rhs.cpu()).to(lhs.device)
