"""Nearest 2x upsampling on the xdna device (the style generator's decoder): the HIP
kernels against PyTorch's own kernels on the same bf16 data.  The forward is a copy
(bit-exact with PyTorch's CPU kernel); the backward sums each 2x2 block of dy in fp32 in
row-major order and rounds once, which is PyTorch-ROCm's order (bit-exact with its GPU
kernel) and within 1 bf16 ulp of the float64 sum."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
import xdna_train
from xdna_train import hip_abi

pytestmark = pytest.mark.gpu
X = torch.device("xdna")


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("shape", [(40, 64, 9, 9), (2, 3, 5, 7), (1, 1, 1, 1), (3, 32, 18, 18)])
@pytest.mark.parametrize("how", ["scale", "size"])
def test_upsample_nearest2x_matches_pytorch(shape, how):
    g = torch.Generator().manual_seed(sum(shape))
    x = (torch.randn(shape, generator=g) * 4).bfloat16()
    B, C, H, W = shape
    dy = (torch.randn(B, C, 2 * H, 2 * W, generator=g) * 3).bfloat16()
    kw = {"scale_factor": 2} if how == "scale" else {"size": (2 * H, 2 * W)}
    ref_cpu = F.interpolate(x, mode="nearest", **kw)
    # PyTorch-ROCm's backward kernel called directly (autograd on cuda tensors is not used
    # in a process whose accelerator is the xdna backend)
    ref_grad = torch.ops.aten.upsample_nearest2d_backward(dy.cuda(), [2 * H, 2 * W], [B, C, H, W], None, None)
    xd = x.to(X).requires_grad_(True)
    xdna_train.reset_mapped_cpu_stats()
    yd = F.interpolate(xd, mode="nearest", **kw)
    yd.backward(dy.to(X))
    torch.xdna.synchronize()
    stats = xdna_train.mapped_cpu_stats()
    assert stats.get("hip_upsample_nearest2x.fwd.run", {}).get("calls", 0) == 1, stats
    assert stats.get("hip_upsample_nearest2x.bwd.run", {}).get("calls", 0) == 1, stats
    assert np.array_equal(bits(yd), bits(ref_cpu))
    assert np.array_equal(bits(xd.grad), bits(ref_grad))
    # float64 2x2 sums, rounded once: within 1 bf16 ulp
    d = dy.double().numpy().reshape(B, C, H, 2, W, 2).sum(axis=(3, 5))
    got = oracle.bf16_value(bits(xd.grad)).astype(np.float64)
    assert np.all(np.abs(got - d) <= oracle.bf16_ulp(d))


def test_upsample_other_forms_fall_back():
    x = torch.randn(2, 4, 6, 6).bfloat16()
    for kw in ({"scale_factor": 3, "mode": "nearest"}, {"scale_factor": 2, "mode": "bilinear"}):
        ref = F.interpolate(x.cuda(), **kw).cpu()
        xdna_train.reset_mapped_cpu_stats()
        out = F.interpolate(x.to(X), **kw)
        torch.xdna.synchronize()
        stats = xdna_train.mapped_cpu_stats()
        assert "hip_upsample_nearest2x.fwd.run" not in stats, stats
        assert np.array_equal(bits(out), bits(ref))


def test_upsample_c_abi_and_errors():
    lib = hip_abi.load()
    st = torch.cuda.current_stream().cuda_stream
    x = torch.randn(3, 5, 4, 6, device="cuda").bfloat16()
    y = torch.empty(3, 5, 8, 12, device="cuda", dtype=torch.bfloat16)
    assert lib.xdna_upsample_nearest2x_bf16(x.data_ptr(), y.data_ptr(), 15, 4, 6, st) == 0
    dx = torch.empty_like(x)
    assert lib.xdna_upsample_nearest2x_bwd_bf16(y.data_ptr(), dx.data_ptr(), 15, 4, 6, st) == 0
    torch.cuda.synchronize()
    assert torch.equal(y, x.repeat_interleave(2, 2).repeat_interleave(2, 3))
    assert torch.equal(dx.float(), (4 * x.float()).bfloat16().float())
    # misaligned destination: refused on the host
    assert lib.xdna_upsample_nearest2x_bf16(x.data_ptr(), y.data_ptr() + 2, 15, 4, 6, st) == -1
    assert b"aligned" in lib.xdna_hip_last_error()
    assert lib.xdna_upsample_nearest2x_bf16(x.data_ptr(), y.data_ptr(), -1, 4, 6, st) == -1
