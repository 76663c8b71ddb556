"""Column sums (xdna_colsum_bf16, the Linear bias gradient: aten::sum over dim 0 of a 2-D
bf16 tensor) against float64 sums of the same bf16 values: within 2 bf16 ulp (floored at
2^-8 of the largest magnitude) and relative L2 <= 1e-2; the same bits on every run (fixed
order); both the four-column vector form and the one-column form (N % 4 != 0), one row
slice and many.  Through aten: x.sum(0) (keepdim or not) and nn.Linear's bias gradient take
the kernel; other sums keep PyTorch-ROCm's."""
import numpy as np
import pytest
import torch

import oracle
import xdna_train
from gpu_util import check_bf16, dev, dev_zeros, host, ptr, stream

pytestmark = pytest.mark.gpu
X = torch.device("xdna")


@pytest.mark.parametrize("R,N", [(8192, 4096), (8192, 1024), (3, 5), (1, 7), (100, 8), (4096, 1002), (33, 4)])
def test_colsum_matches_fp64(hip, R, N):
    rng = np.random.default_rng(R * 7 + N)
    x = oracle.rng_bf16(rng, (R, N))
    dx = dev(x)
    wb = hip.xdna_colsum_workspace_bytes(ptr(dx), R, N)
    ws = dev_zeros((max(1, wb // 2),)) if wb else None
    out = dev_zeros((N,))
    assert hip.xdna_colsum_bf16(ptr(dx), ptr(out), R, N, ptr(ws), wb, stream()) == 0
    got = host(out)
    check_bf16(got, oracle.bf16_value(x).astype(np.float64).sum(0), what=f"colsum {R}x{N}")
    out2 = dev_zeros((N,))
    assert hip.xdna_colsum_bf16(ptr(dx), ptr(out2), R, N, ptr(ws), wb, stream()) == 0
    np.testing.assert_array_equal(host(out2), got)
    if wb:
        assert hip.xdna_colsum_bf16(ptr(dx), ptr(out2), R, N, ptr(ws), wb - 1, stream()) == -1


def _calls(name):
    return xdna_train.mapped_cpu_stats().get(name, {}).get("calls", 0)


def test_aten_sum_rows_and_linear_bias_grad():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(257, 96, generator=g).bfloat16()
    xd = x.to(X)
    xdna_train.reset_mapped_cpu_stats()
    s0 = xd.sum(0)
    s1 = xd.sum(dim=0, keepdim=True)
    s2 = xd.sum(1)  # other sums: PyTorch-ROCm
    xdna_train.synchronize()
    assert _calls("hip_colsum.run") == 2
    ref = x.double().sum(0).numpy()
    bits = lambda t: t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    check_bf16(bits(s0), ref, what="sum(0)")
    assert s1.shape == (1, 96) and torch.equal(s1.cpu().view(-1), s0.cpu())
    assert torch.allclose(s2.cpu().float(), x.float().sum(1), rtol=2e-2, atol=2e-2)
    # Linear's bias gradient
    torch.manual_seed(0)
    lin = torch.nn.Linear(96, 64).bfloat16().to(X)
    inp = torch.randn(257, 96, generator=g).bfloat16()
    dy = torch.randn(257, 64, generator=g).bfloat16()
    xdna_train.reset_mapped_cpu_stats()
    lin(inp.to(X)).backward(dy.to(X))
    xdna_train.synchronize()
    assert _calls("hip_colsum.run") == 1
    check_bf16(bits(lin.bias.grad), dy.double().sum(0).numpy(), what="linear bias grad")
