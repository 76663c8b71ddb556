"""ctypes binding of the C ABI in ``include/xdna_hip.h`` (``_lib/libxdna_hip.so``).

The PrivateUse1 backend calls the same entry points from C++; this binding serves
Python callers, benchmarks and the tests, mirroring how the reference's tests bind its
host packing library (tests/run_conv3x3w_pack.py:16-27).  ``load()`` raises if the
library was not built: there is no CPU substitute for any of these kernels.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libxdna_hip.so"

P = ctypes.c_void_p
I = ctypes.c_int
L = ctypes.c_int64
Z = ctypes.c_size_t
F = ctypes.c_float
D = ctypes.c_double
PP = ctypes.POINTER(ctypes.c_void_p)
PL = ctypes.POINTER(ctypes.c_int64)

# row layouts of the packed conv operands (XDNA_CONV3X3_LAYOUT_*)
LAYOUT_REF = 0
LAYOUT_TIGHT = 1

# name -> (restype, argtypes); every function declared in include/xdna_hip.h.
SIGNATURES = {
    "xdna_hip_last_error": (ctypes.c_char_p, []),
    "xdna_hip_poisoned": (I, []),
    "xdna_hip_inject_failure": (I, [L, I]),
    "xdna_hip_reset_failure_state": (I, []),
    "xdna_hip_launch_count": (L, []),
    "xdna_hip_device_count": (I, []),
    "xdna_hip_set_device": (I, [I]),
    "xdna_hip_get_device": (I, [ctypes.POINTER(I)]),
    "xdna_hip_device_properties": (I, [ctypes.c_char_p, Z, ctypes.POINTER(I), ctypes.POINTER(Z),
                                       ctypes.POINTER(I)]),
    "xdna_hip_malloc": (P, [Z]),
    "xdna_hip_free": (I, [P]),
    "xdna_hip_cache_alloc": (P, [Z]),
    "xdna_hip_cache_free": (I, [P]),
    "xdna_hip_cache_empty": (I, []),
    "xdna_hip_cache_stats": (I, [PL, I]),
    "xdna_hip_cache_pool_create": (L, []),
    "xdna_hip_cache_pool_begin": (I, [L]),
    "xdna_hip_cache_pool_end": (I, []),
    "xdna_hip_cache_pool_release": (I, [L]),
    "xdna_round_bf16": (I, [P, P, L, P]),
    "xdna_hip_memcpy_async": (I, [P, P, Z, I, P]),
    "xdna_hip_memset_async": (I, [P, I, Z, P]),
    "xdna_hip_stream_synchronize": (I, [P]),
    "xdna_hip_device_synchronize": (I, []),
    "xdna_hip_event_create": (P, [I]),
    "xdna_hip_event_destroy": (I, [P]),
    "xdna_hip_event_record": (I, [P, P]),
    "xdna_hip_event_synchronize": (I, [P]),
    "xdna_hip_event_query": (I, [P]),
    "xdna_hip_event_elapsed_ms": (I, [P, P, ctypes.POINTER(F)]),
    "xdna_hip_stream_wait_event": (I, [P, P]),
    "xdna_hip_stream_create": (P, []),
    "xdna_hip_cache_pool_current": (L, []),
    "xdna_hip_stream_capturing": (I, [P]),
    "xdna_hip_set_wait_timeout_ms": (I, [L]),
    "xdna_hip_wait_timeout_ms": (L, []),
    "xdna_hip_max_wait_ms": (D, []),
    "xdna_hip_inject_wait_timeout": (I, [L]),
    "xdna_conv3x3w_pack_input_bf16": (I, [P, P, I, I, I, I, I, P]),
    "xdna_conv3x3w_pack_input_range_bf16": (I, [P, P, I, I, I, I, I, I, I, P]),
    "xdna_conv3x3w_pack_input_strips_range_bf16": (I, [P, P, I, I, I, I, I, I, I, I, I, I, P]),
    "xdna_conv3x3w_pack_input_dense_bf16": (I, [P, P, I, I, I, I, P]),
    "xdna_conv3x3w_pack_weights_bfp16": (I, [P, P, I, I, I, I, P]),
    "xdna_conv3x3w_pack_weights_dx_bfp16": (I, [P, P, I, I, I, I, P]),
    "xdna_conv3x3w_weights_bfp16_bytes": (Z, [I]),
    "xdna_bfp16_decode_f32": (I, [P, P, L, P]),
    "xdna_bfp16_quantize8_bf16": (I, [P, P, L, P]),
    "xdna_conv3x3_layout_rows_stride2_bf16": (I, [P, P, P, P, I, I, I, I, I, I, P]),
    "xdna_conv3x3_layout_pack_dilate2_bf16": (I, [P, P, I, I, I, I, I, P]),
    "xdna_conv3x3_layout_rows_bfp16_emul_bf16": (I, [P, P, P, P, I, I, I, I, I, I, I, P]),
    "xdna_conv2d_fwd_bf16": (I, [P, P, P, P] + [I] * 11 + [P]),
    "xdna_instance_norm_fwd_bf16": (I, [P, P, P, I, P, P, P, L, L, L, ctypes.c_double, P]),
    "xdna_instance_norm_bwd_bf16": (I, [P, P, P, I, P, P, P, P, P, L, L, L, P]),
    "xdna_instance_norm_act_fwd_bf16": (I, [P, P, P, I, P, P, P, L, L, L, D, I, F, P]),
    "xdna_instance_norm_act_bwd_bf16": (I, [P, P, P, P, I, P, P, P, P, P, L, L, L, I, F, P]),
    "xdna_upsample_nearest2x_bf16": (I, [P, P, L, I, I, P]),
    "xdna_conv2d_set_variant": (I, [I]),
    "xdna_subsample2_bf16": (I, [P, P, L, I, I, P]),
    "xdna_conv3x3_prepare_weights_both_bf16": (I, [P, P, P, I, I, P]),
    "xdna_conv3x3_wgrad_rows_workspace_bytes": (Z, [I, I, I, I, I, I]),
    "xdna_conv3x3_wgrad_rows_bf16": (I, [P, P, P, P, I, I, I, I, I, I, P, Z, P]),
    "xdna_conv3x3_set_wgrad_rows_kt": (I, [I]),
    "xdna_conv3x3_set_wgrad_rows_kernel": (I, [I]),
    "xdna_dilate2_bf16": (I, [P, P, L, I, I, P]),
    "xdna_upsample_nearest2x_bwd_bf16": (I, [P, P, L, I, I, P]),
    "xdna_conv2d_dgrad_bf16": (I, [P, P, P] + [I] * 11 + [P]),
    "xdna_conv2d_wgrad_bf16": (I, [P, P, P, P] + [I] * 11 + [P]),
    "xdna_conv3x3w_unpack_output_bf16": (I, [P, P, I, I, I, I, I, I, P]),
    "xdna_conv3x3w_unpack_output_range_bf16": (I, [P, P, I, I, I, I, I, I, I, I, P]),
    "xdna_conv3x3w_unpack_output_strips_range_bf16": (I, [P, P, I, I, I, I, I, I, I, I, I, I, P]),
    "xdna_conv3x3w_geometry": (I, [I, I, I, I, PL]),
    "xdna_conv3x3_fwd_workspace_bytes": (Z, [I, I, I, I, I]),
    "xdna_conv3x3_fwd_bf16": (I, [P, P, P, P, I, I, I, I, I, P, Z, P]),
    "xdna_conv3x3_dgrad_workspace_bytes": (Z, [I, I, I, I, I]),
    "xdna_conv3x3_dgrad_bf16": (I, [P, P, P, I, I, I, I, I, P, Z, P]),
    "xdna_conv3x3_wgrad_workspace_bytes": (Z, [I, I, I, I, I]),
    "xdna_conv3x3_wgrad_bf16": (I, [P, P, P, P, I, I, I, I, I, P, Z, P]),
    "xdna_conv3x3_bias_grad_bf16": (I, [P, P, I, I, I, I, P]),
    "xdna_conv3x3w_packed_bytes": (Z, [I, I, I, I]),
    "xdna_conv3x3_prepared_weight_bytes": (Z, [I, I]),
    "xdna_conv3x3_prepare_weights_bf16": (I, [P, P, I, I, I, P]),
    "xdna_conv3x3_set_rows_variant": (I, [I]),
    "xdna_conv3x3_rows_bf16": (I, [P, P, P, P, I, I, I, I, I, P]),
    "xdna_conv3x3_layout_packed_bytes": (Z, [I, I, I, I, I]),
    "xdna_conv3x3_layout_pack_bf16": (I, [P, P, I, I, I, I, I, P]),
    "xdna_conv3x3_layout_rows_bf16": (I, [P, P, P, P, I, I, I, I, I, I, P]),
    "xdna_conv3x3_layout_rows_act_bf16": (I, [P, P, P, P, I, I, I, I, I, I, I, P]),
    "xdna_conv3x3_nchw_small_eligible": (I, [I, I, I, I, I]),
    "xdna_conv3x3_nchw_act_bf16": (I, [P, P, P, P, I, I, I, I, I, I, I, P]),
    "xdna_region_maxpool2_bf16": (I, [P, P, L, I, I, P]),
    "xdna_region_backward_bf16": (I, [P, P, P, P, P, P, P, F, P, I, P, L, I, I, P]),
    "xdna_region_loss_parts": (I, []),
    "xdna_region_sqdiff_bf16": (I, [P, P, L, F, P, P]),
    "xdna_region_gram_sqdiff_bf16": (I, [P, P, L, L, L, F, F, P, P]),
    "xdna_region_loss_finish": (I, [P, I, P, P, P]),
    "xdna_region_gram_grad_bf16": (I, [P, P, L, L, I, F, F, P, I, P, P]),
    "xdna_mse_loss_workspace_bytes": (Z, [L]),
    "xdna_mse_loss": (I, [P, P, I, L, L, I, P, P, Z, P]),
    "xdna_mse_loss_bwd": (I, [P, I, P, P, I, L, L, I, P, P]),
    "xdna_colsum_workspace_bytes": (Z, [P, L, L]),
    "xdna_colsum_bf16": (I, [P, P, L, L, P, Z, P]),
    "xdna_conv3x3_wgrad_pack_bf16": (I, [P, P, I, I, I, I, I, P, Z, P]),
    "xdna_conv3x3_wgrad_packed_bf16": (I, [P, P, I, I, I, I, I, P, Z, P]),
    "xdna_gemm_set_variant": (I, [I]),
    "xdna_gemm_set_small": (I, [I]),
    "xdna_conv3x3_set_pack_rows": (I, [I]),
    "xdna_conv3x3_set_prep_tile": (I, [I]),
    "xdna_conv3x3_prepare_weights_multi_bf16": (I, [I, P, P, P, P, P, P]),
    "xdna_conv3x3_set_wgrad_splits": (I, [I]),
    "xdna_conv3x3_set_wgrad_tile": (I, [I]),
    "xdna_gemm_bf16": (I, [P, P, P, P, I, I, I, I, L, L, L, L, L, L, L, L, L, I, L, L, F, F, P]),
    "xdna_gemm_bf16_noalloc": (I, [P, P, P, P, I, I, I, I, L, L, L, L, L, L, L, L, L, I, L, L, F, F, P]),
    "xdna_batch_norm_fwd_bf16": (I, [P, P, P, I, P, P, P, L, L, L, D, P]),
    "xdna_batch_norm_train_fwd_bf16": (I, [P, P, P, I, P, P, I, D, D, P, P, P, L, L, L, P]),
    "xdna_batch_norm_train_bwd_bf16": (I, [P, P, P, I, P, P, P, P, P, L, L, L, P]),
    "xdna_batch_norm_train_act_fwd_bf16": (I, [P, P, P, I, P, P, I, D, D, P, P, P, L, L, L, I, F, P]),
    "xdna_batch_norm_train_act_bwd_bf16": (I, [P, P, P, P, I, P, P, P, P, P, L, L, L, I, F, P]),
    "xdna_batch_norm_bwd_bf16": (I, [P, P, P, I, P, P, P, P, P, L, L, L, P]),
    "xdna_foreach_add_scalar_f32": (I, [I, PP, PL, ctypes.c_float, P]),
    "xdna_fused_adam": (I, [I, PP, PP, PP, PP, PP, PP, PL, I, D, D, D, D, D, I, I, I, P, P, P]),
    "xdna_fused_adam_tensor_lr": (I, [I, PP, PP, PP, PP, PP, PP, PL, I, P, I, D, D, D, D, I, I, I, P, P, P]),
}

_lib = None


class HipError(RuntimeError):
    pass


def load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise HipError(
                f"{LIB_PATH} is missing: build it with "
                "`python pytorch-xdna2_amd/build_native.py` (no CPU fallback exists)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def last_error() -> str:
    return load().xdna_hip_last_error().decode()


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        raise HipError(f"{what or 'xdna_hip'} failed: {last_error()}")


def ptr_array(ptrs) -> ctypes.Array:
    arr = (ctypes.c_void_p * len(ptrs))()
    for i, p in enumerate(ptrs):
        arr[i] = p
    return arr


def int64_array(vals) -> ctypes.Array:
    arr = (ctypes.c_int64 * len(vals))()
    for i, v in enumerate(vals):
        arr[i] = int(v)
    return arr
