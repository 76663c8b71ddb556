"""1x1 convolutions (stride 1 and 2, no padding: ResNet's downsampling shortcut) on the
HIP GEMM path through aten.convolution(_backward): forward, input, weight and bias
gradients against the float64 oracle (oracle.conv2d_*, pinned by brute force and
PyTorch's CPU conv in tests/test_oracle_conv2d.py), with the conv bar (2 bf16 ulp with the
ulp(max|ref| 2^-8) floor, relative L2 <= 1e-2), on odd sizes and at BASELINE config 5's
full shapes.  Path counters prove the HIP path ran (no MIOpen)."""
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


@pytest.mark.parametrize("B,Ci,Co,H,W,s,bias", [
    (4, 64, 128, 16, 16, 2, False),
    (3, 32, 48, 9, 7, 2, True),      # odd planes: ceil(H/2) outputs
    (2, 128, 64, 8, 8, 1, True),
    (5, 24, 40, 5, 11, 1, False),
    (128, 64, 128, 64, 64, 2, False),   # config 5 shortcuts
    (128, 128, 256, 32, 32, 2, False),
    (128, 256, 512, 16, 16, 2, False),
])
def test_conv1x1_matches_oracle(B, Ci, Co, H, W, s, bias):
    print(f"conv1x1 B{B} {Ci}->{Co} {H}x{W} s{s} bias={bias}", flush=True)
    g = torch.Generator().manual_seed(B * 7 + Ci + s)
    x = torch.randn(B, Ci, H, W, generator=g).bfloat16()
    w = (torch.randn(Co, Ci, 1, 1, generator=g) / Ci ** 0.5).bfloat16()
    b = (torch.randn(Co, generator=g) * 0.1).bfloat16() if bias else None
    Ho, Wo = (H - 1) // s + 1, (W - 1) // s + 1
    dy = torch.randn(B, Co, Ho, Wo, generator=g).bfloat16()
    xd = x.to(X).requires_grad_()
    wd = w.to(X).requires_grad_()
    bd = b.to(X).requires_grad_() if bias else None
    xdna_train.reset_mapped_cpu_stats()
    y = torch.nn.functional.conv2d(xd, wd, bd, stride=s)
    y.backward(dy.to(X))
    st = xdna_train.mapped_cpu_stats()
    for k in ("hip_conv1x1.fwd.run", "hip_conv1x1.bwd.run"):
        assert st.get(k, {}).get("calls", 0) == 1, (k, st)
    assert not any(k.startswith("aten::convolution") for k in st), st
    xb, wb, dyb = bits(x), bits(w), bits(dy)
    bb = bits(b) if bias else None
    check_bf16(bits(y), oracle.conv2d_fwd(xb, wb, bb, stride=(s, s)), what="1x1 fwd")
    check_bf16(bits(xd.grad), oracle.conv2d_dgrad(dyb, wb, (H, W), stride=(s, s)), what="1x1 dgrad")
    gw, gb = oracle.conv2d_wgrad(xb, dyb, (1, 1), stride=(s, s))
    check_bf16(bits(wd.grad), gw, what="1x1 wgrad")
    if bias:
        check_bf16(bits(bd.grad), gb, what="1x1 bias grad")
