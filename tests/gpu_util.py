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


# ---------------------------------------------------------------------------------------
# Full-tensor checks on the device (tensors too large for host numpy)
# ---------------------------------------------------------------------------------------
def bf16_ulp_dev(x: torch.Tensor) -> torch.Tensor:
    """oracle.bf16_ulp on the device: 2^(floor(log2 |x|) - 7), |x| floored at the
    smallest normal fp32."""
    a = x.abs().to(torch.float64).clamp_min(float(np.finfo(np.float32).tiny))
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


def check_bf16_dev(got: torch.Tensor, ref: torch.Tensor, ulps: float = 2.0, rel_l2: float = 1e-2,
                   what: str = "") -> float:
    """check_bf16's bar (elementwise ulps with the ulp(max|ref| 2^-8) floor, relative L2)
    computed on the GPU.  `got`: bf16 ROCm tensor; `ref`: float32/64 ROCm tensor."""
    g = got.to(torch.float64)
    r = ref.to(torch.float64)
    assert g.shape == r.shape, (g.shape, r.shape)
    assert bool(torch.isfinite(g).all()), f"{what}: non-finite output"
    amax = float(r.abs().max()) if r.numel() else 0.0
    floor = float(bf16_ulp_dev(torch.tensor(amax * 2.0 ** -8))) if amax > 0 else 0.0
    unit = bf16_ulp_dev(r).clamp_min(floor)
    ratio = (g - r).abs() / unit
    worst = float(ratio.max()) if ratio.numel() else 0.0
    if worst > ulps:
        i = int(ratio.argmax())
        nbad = int((ratio > ulps).sum())
        raise AssertionError(f"{what}: {nbad}/{ratio.numel()} elements beyond {ulps} bf16 ulp; worst at flat "
                             f"{i}: got {float(g.flatten()[i])!r} ref {float(r.flatten()[i])!r} ({worst:.2f} ulp)")
    nrm = float(r.norm())
    if nrm > 0:
        rel = float((g - r).norm()) / nrm
        assert rel <= rel_l2, f"{what}: relative L2 {rel:.3e} > {rel_l2}"
    return worst


def conv3x3_ref_fp32_dev(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None, dy: torch.Tensor,
                         chunk_bytes: int = 1 << 30):
    """fp32 reference of a 3x3 / stride-1 / pad-1 conv's forward, input gradient, weight
    gradient and bias gradient on ROCm tensors, as im2col GEMMs (F.unfold / F.fold and
    fp32 matmuls, no MIOpen), over chunks of images."""
    import torch.nn.functional as F

    N, Ci, H, W = x.shape
    Co = w.shape[0]
    w2 = w.float().reshape(Co, Ci * 9)
    per_img = Ci * 9 * H * W * 4
    step = max(1, min(N, chunk_bytes // max(1, per_img)))
    y = torch.empty(N, Co, H, W, device=x.device, dtype=torch.float32)
    dx = torch.empty(N, Ci, H, W, device=x.device, dtype=torch.float32)
    gw = torch.zeros(Co, Ci * 9, device=x.device, dtype=torch.float64)
    for n0 in range(0, N, step):
        n1 = min(N, n0 + step)
        cols = F.unfold(x[n0:n1].float(), 3, padding=1)             # [n, Ci*9, HW]
        yc = torch.matmul(w2, cols)                                  # [n, Co, HW]
        if b is not None:
            yc += b.float().view(1, Co, 1)
        y[n0:n1] = yc.view(n1 - n0, Co, H, W)
        d = dy[n0:n1].float().reshape(n1 - n0, Co, H * W)
        dx[n0:n1] = F.fold(torch.matmul(w2.t(), d), (H, W), 3, padding=1)
        gw += torch.matmul(d, cols.transpose(1, 2)).sum(0, dtype=torch.float64)
    gb = dy.to(torch.float64).sum((0, 2, 3))
    return y, dx, gw.view(Co, Ci, 3, 3), gb
