"""MI355X-native ``xdna`` PyTorch device: the training hot path of torch-xdna2 (3x3 bf16
conv forward / dgrad / wgrad, mm / addmm / bmm, fused Adam, conv3x3w layout packing)
as hand-written gfx950 HIP kernels behind the reference's PrivateUse1 operator surface.
Importing registers the device, as the reference does (xdna_train/__init__.py:27)."""

from .device import (
    allocator_stats,
    async_dw_stats,
    autotune_result,
    bfp16_emulation,
    bo_handle,
    conv_layout,
    coherency_state,
    empty_cache,
    fallback_stats,
    general_conv_mode,
    is_available,
    is_xrt_backed,
    mapped_cpu_stats,
    max_wait_ms,
    native_library_path,
    npu_mode,
    register_xdna_device,
    reset_fallback_stats,
    reset_mapped_cpu_stats,
    set_bfp16_emulation,
    set_general_conv_mode,
    set_conv_layout,
    set_npu_mode,
    set_wait_timeout_ms,
    set_wgrad_form,
    synchronize,
    try_register_xdna_device,
    wait_for_builds,
    wgrad_form,
)

from .graphs import Graph, graph

__version__ = "0.1.0"

try_register_xdna_device()

__all__ = [
    "__version__",
    "register_xdna_device",
    "try_register_xdna_device",
    "is_available",
    "synchronize",
    "empty_cache",
    "allocator_stats",
    "async_dw_stats",
    "autotune_result",
    "set_npu_mode",
    "npu_mode",
    "set_general_conv_mode",
    "general_conv_mode",
    "set_wgrad_form",
    "set_conv_layout",
    "conv_layout",
    "set_bfp16_emulation",
    "bfp16_emulation",
    "wgrad_form",
    "wait_for_builds",
    "set_wait_timeout_ms",
    "max_wait_ms",
    "reset_fallback_stats",
    "fallback_stats",
    "mapped_cpu_stats",
    "reset_mapped_cpu_stats",
    "native_library_path",
    "is_xrt_backed",
    "bo_handle",
    "coherency_state",
    "Graph",
    "graph",
]
