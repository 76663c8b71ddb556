"""3x3 / stride-2 / pad-1 convs on the xdna device, run through the stride-1 conv kernels
(forward = every other output of the stride-1 conv; gradients = the stride-1 gradients
of the gradient spread onto the stride-1 grid with zeros), against the float64 oracle of
the strided conv, to the conv bar: 2 bf16 ulp (floor at ulp(max|ref| * 2^-8)) and
relative L2 <= 1e-2.  Shapes: the style encoder's two strided layers, ResNet's
downsampling conv, odd sizes (ceil(H/2) outputs) and non-square images."""
import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
import xdna_train
from gpu_util import check_bf16
from xdna_train import hip_abi

pytestmark = pytest.mark.gpu
X = torch.device("xdna")


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("shape", [(4, 32, 64, 36, 36), (4, 64, 128, 18, 18), (2, 64, 128, 16, 16),
                                   (3, 5, 7, 13, 11), (1, 3, 64, 9, 20)])
def test_stride2_conv_matches_oracle(shape):
    B, cin, cout, H, W = shape
    print(f"conv3x3 s2 {shape}", flush=True)
    torch.manual_seed(sum(shape))
    conv = nn.Conv2d(cin, cout, 3, stride=2, padding=1).bfloat16()
    x = torch.randn(B, cin, H, W).bfloat16()
    cd = nn.Conv2d(cin, cout, 3, stride=2, padding=1).bfloat16().to(X)
    cd.load_state_dict(conv.state_dict())
    xdna_train.reset_mapped_cpu_stats()
    xd = x.to(X).requires_grad_()
    yd = cd(xd)
    assert yd.shape == (B, cout, (H + 1) // 2, (W + 1) // 2)
    dy = torch.randn(yd.shape).bfloat16()
    yd.backward(dy.to(X))
    torch.xdna.synchronize()
    st = xdna_train.mapped_cpu_stats()
    assert st.get("hip_conv3x3_s2.fwd.run", {}).get("calls", 0) == 1, st
    assert st.get("hip_conv3x3_s2.bwd.run", {}).get("calls", 0) == 1, st
    assert "aten::convolution.rocm" not in st and "aten::convolution_backward.rocm" not in st, st
    xb, wb, bb, dyb = (bits(t) for t in (x, conv.weight, conv.bias, dy))
    check_bf16(bits(yd), oracle.conv2d_fwd(xb, wb, bb, (2, 2), (1, 1)), what=f"fwd {shape}")
    check_bf16(bits(xd.grad), oracle.conv2d_dgrad(dyb, wb, (H, W), (2, 2), (1, 1)), what=f"dgrad {shape}")
    gw, gb = oracle.conv2d_wgrad(xb, dyb, (3, 3), (2, 2), (1, 1))
    check_bf16(bits(cd.weight.grad), gw, what=f"wgrad {shape}")
    check_bf16(bits(cd.bias.grad), gb, what=f"bias grad {shape}")


@pytest.mark.parametrize("H,W", [(7, 10), (16, 16), (9, 12), (36, 36), (64, 64), (5, 4)])
def test_stride2_sampling_c_abi(H, W):
    """Both samplings bit for bit against slicing, in the element form (W % 4 != 0) and the
    vector form (W % 4 == 0, odd H included)."""
    lib = hip_abi.load()
    st = torch.cuda.current_stream().cuda_stream
    Ho, Wo = (H + 1) // 2, (W + 1) // 2
    full = torch.randn(3, 4, H, W, device="cuda").bfloat16()
    y = torch.full((3, 4, Ho, Wo), 7.0, device="cuda").bfloat16()
    assert lib.xdna_subsample2_bf16(full.data_ptr(), y.data_ptr(), 12, H, W, st) == 0
    back = torch.full((3, 4, H, W), 7.0, device="cuda").bfloat16()
    assert lib.xdna_dilate2_bf16(y.data_ptr(), back.data_ptr(), 12, H, W, st) == 0
    torch.cuda.synchronize()
    assert torch.equal(y, full[:, :, ::2, ::2])
    ref = torch.zeros_like(full)
    ref[:, :, ::2, ::2] = full[:, :, ::2, ::2]
    assert torch.equal(back, ref)
    assert lib.xdna_subsample2_bf16(full.data_ptr(), None, 12, H, W, st) == -1
