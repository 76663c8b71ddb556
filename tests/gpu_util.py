"""Helpers of the GPU tests: device buffers (torch for memory only) and the bf16
parity check used for conv and GEMM results."""
from __future__ import annotations

import numpy as np
import torch

import oracle


def dev(bits: np.ndarray) -> torch.Tensor:
    """uint16 numpy -> int16 device tensor with the same bits."""
    a = np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)
    return torch.from_numpy(a.copy()).cuda()


def dev_zeros(shape, dtype=torch.int16) -> torch.Tensor:
    return torch.zeros(shape, dtype=dtype, device="cuda")


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.uint16) if t.dtype in (torch.int16, torch.bfloat16) else t.cpu().numpy()


def ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def check_bf16(got_bits: np.ndarray, ref: np.ndarray, ulps: float = 2.0, rel_l2: float = 1e-2,
               what: str = ""):
    """Parity bar for bf16 results of fp32-accumulated sums:
    |got - ref| <= ulps * max(ulp(ref), ulp(max|ref| * 2^-8)) elementwise (the floor covers
    outputs that cancel to near zero), and ||got - ref|| / ||ref|| <= rel_l2."""
    got = oracle.bf16_value(got_bits).astype(np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    amax = float(np.max(np.abs(ref))) if ref.size else 0.0
    floor = oracle.bf16_ulp(amax * 2.0 ** -8) if amax > 0 else 0.0
    tol = ulps * np.maximum(oracle.bf16_ulp(ref), floor)
    err = np.abs(got - ref)
    bad = err > tol
    if bad.any():
        i = np.unravel_index(np.argmax(err / np.maximum(tol, 1e-300)), err.shape)
        raise AssertionError(f"{what}: {int(bad.sum())}/{err.size} elements beyond {ulps} bf16 ulp; "
                             f"worst at {i}: got {got[i]!r} ref {ref[i]!r} tol {tol[i]!r}")
    nrm = float(np.linalg.norm(ref))
    if nrm > 0:
        rel = float(np.linalg.norm(got - ref)) / nrm
        assert rel <= rel_l2, f"{what}: relative L2 {rel:.3e} > {rel_l2}"
    return float(np.max(err / np.maximum(oracle.bf16_ulp(ref), floor))) if ref.size else 0.0
