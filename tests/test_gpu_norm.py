"""InstanceNorm on the xdna device: the HIP batch-norm kernels (reached through
native_batch_norm / native_batch_norm_backward, as PyTorch's instance_norm calls them)
against an fp64 autograd reference computed from the same bf16 inputs on the CPU.
Tolerance: bf16 outputs within 2 bf16 ulp (floor at 2^-8 of the largest magnitude) and
relative L2 <= 1e-2; fp32 statistics within 1e-5 relative."""
import numpy as np
import pytest
import torch

import oracle
import xdna_train
from gpu_util import check_bf16

pytestmark = pytest.mark.gpu
X = torch.device("xdna")


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("shape,affine,pdtype", [
    ((40, 128, 9, 9), True, torch.bfloat16),
    ((40, 32, 36, 36), True, torch.bfloat16),
    ((2, 3, 5, 7), False, torch.bfloat16),
    ((3, 5, 1, 2), True, torch.float32),
    ((1, 4, 130, 130), True, torch.bfloat16),
])
def test_instance_norm_matches_fp64(shape, affine, pdtype):
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(shape, generator=g) * 3 + 0.5).bfloat16()
    dy = torch.randn(shape, generator=g).bfloat16()
    C = shape[1]
    w = (torch.rand(C, generator=g) + 0.5).to(pdtype) if affine else None
    b = (torch.randn(C, generator=g) * 0.1).to(pdtype) if affine else None
    # reference: fp64 instance norm of the bf16 inputs
    xr = x.double().requires_grad_(True)
    wr = w.double().requires_grad_(True) if affine else None
    br = b.double().requires_grad_(True) if affine else None
    yr = torch.nn.functional.instance_norm(xr, weight=wr, bias=br, eps=1e-5)
    yr.backward(dy.double())
    # device
    xd = x.to(X).requires_grad_(True)
    wd = w.to(X).requires_grad_(True) if affine else None
    bd = b.to(X).requires_grad_(True) if affine else None
    xdna_train.reset_mapped_cpu_stats()
    yd = torch.nn.functional.instance_norm(xd, weight=wd, bias=bd, eps=1e-5)
    yd.backward(dy.to(X))
    torch.xdna.synchronize()
    stats = xdna_train.mapped_cpu_stats()
    assert stats.get("hip_batch_norm.fwd.run", {}).get("calls", 0) == 1, stats
    assert stats.get("hip_batch_norm.bwd.run", {}).get("calls", 0) == 1, stats
    check_bf16(bits(yd), yr.detach().numpy(), what="instance_norm out")
    check_bf16(bits(xd.grad), xr.grad.numpy(), what="instance_norm dx")
    if affine:
        for got, ref, name in ((wd.grad, wr.grad, "dweight"), (bd.grad, br.grad, "dbias")):
            gv = got.detach().cpu().double().numpy()
            rv = ref.numpy()
            if pdtype == torch.bfloat16:
                # per-image sums rounded to bf16, then summed over the batch by autograd
                tol = shape[0] * 2 * oracle.bf16_ulp(np.abs(rv) + np.abs(ref.numpy()).max() * 2.0 ** -8)
            else:
                tol = 1e-4 * (np.abs(rv) + np.abs(rv).max())
            assert (np.abs(gv - rv) <= tol).all(), (name, np.abs(gv - rv).max(), tol.max())


def test_batch_norm_with_running_stats_falls_back():
    x = torch.randn(4, 8, 6, 6).bfloat16()
    bn = torch.nn.BatchNorm2d(8).bfloat16()
    ref = bn(x.clone())
    bnd = torch.nn.BatchNorm2d(8).bfloat16().to(X)
    xdna_train.reset_mapped_cpu_stats()
    out = bnd(x.to(X))
    torch.xdna.synchronize()
    stats = xdna_train.mapped_cpu_stats()
    assert stats.get("aten::native_batch_norm.rocm", {}).get("calls", 0) >= 1, stats
    assert torch.allclose(out.cpu().float(), ref.float(), atol=3e-2, rtol=3e-2)
