"""3x3 / stride-2 / pad-1 convs on the xdna device, run through the stride-1 conv kernels
(forward = the even outputs of the stride-1 conv, stored straight into the strided
output; gradients = the stride-1 gradients of the gradient spread onto the stride-1 grid
with zeros, packed in one pass), against the float64 oracle of the strided conv, to the
conv bar: 2 bf16 ulp (floor at ulp(max|ref| * 2^-8)) and relative L2 <= 1e-2.  Shapes:
the style encoder's two strided layers, ResNet's downsampling conv, odd sizes (ceil(H/2)
outputs) and non-square images.  The two entry points of that path are checked bit for
bit against the sampling kernels they replace."""
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


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("shape", [(2, 64, 36, 36), (3, 70, 17, 13), (1, 3, 64, 64), (2, 130, 18, 72),
                                   (4, 32, 9, 9), (1, 8, 1, 1), (2, 64, 72, 40)])
def test_spread_pack_is_the_pack_of_the_spread(shape, layout):
    """xdna_conv3x3_layout_pack_dilate2_bf16 writes the same bytes as the ordinary pack of
    the materialized spread (every byte of the buffer: borders, halos, padded channels)."""
    lib = hip_abi.load()
    st = torch.cuda.current_stream().cuda_stream
    B, C, H, W = shape
    print(f"spread pack {shape} layout {layout}", flush=True)
    g = torch.randn(B, C, (H + 1) // 2, (W + 1) // 2, device="cuda").bfloat16()
    full = torch.zeros(B, C, H, W, device="cuda").bfloat16()
    full[:, :, ::2, ::2] = g
    nb = lib.xdna_conv3x3_layout_packed_bytes(B, C, H, W, layout)
    want = torch.full((nb // 2,), 7, dtype=torch.int16, device="cuda")
    got = torch.full((nb // 2,), 9, dtype=torch.int16, device="cuda")
    assert lib.xdna_conv3x3_layout_pack_bf16(full.data_ptr(), want.data_ptr(), B, C, H, W, layout, st) == 0
    assert lib.xdna_conv3x3_layout_pack_dilate2_bf16(g.data_ptr(), got.data_ptr(), B, C, H, W, layout, st) == 0
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.fixture
def rows_variant(request):
    lib = hip_abi.load()
    assert lib.xdna_conv3x3_set_rows_variant(request.param) == 0
    yield request.param
    assert lib.xdna_conv3x3_set_rows_variant(0) == 0


@pytest.mark.parametrize("rows_variant", [0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11], indirect=True, ids=lambda v: f"v{v}")
@pytest.mark.parametrize("shape", [(4, 64, 128, 18, 18), (2, 32, 64, 36, 36), (3, 70, 300, 13, 11), (1, 128, 64, 9, 40)])
def test_stride2_output_is_the_subsampled_stride1_output(shape, rows_variant):
    """xdna_conv3x3_layout_rows_stride2_bf16 stores exactly the even outputs of the
    stride-1 conv (bit for bit against xdna_conv3x3_layout_rows_bf16 + subsample), for
    every rows-kernel variant (the ones without a buffer-store epilogue fall back to the
    automatic choice), split-K small grids included."""
    lib = hip_abi.load()
    st = torch.cuda.current_stream().cuda_stream
    B, cin, cout, H, W = shape
    print(f"stride-2 output {shape} variant {rows_variant}", flush=True)
    torch.manual_seed(sum(shape))
    x = torch.randn(B, cin, H, W, device="cuda").bfloat16()
    w = (torch.randn(cout, cin, 3, 3, device="cuda") * 0.05).bfloat16()
    b = (torch.randn(cout, device="cuda") * 0.1).bfloat16()
    nb = lib.xdna_conv3x3_layout_packed_bytes(B, cin, H, W, 1)
    xp = torch.empty(nb // 2, dtype=torch.int16, device="cuda")
    assert lib.xdna_conv3x3_layout_pack_bf16(x.data_ptr(), xp.data_ptr(), B, cin, H, W, 1, st) == 0
    wt = torch.empty(lib.xdna_conv3x3_prepared_weight_bytes(cin, cout) // 2, dtype=torch.int16, device="cuda")
    assert lib.xdna_conv3x3_prepare_weights_bf16(w.data_ptr(), wt.data_ptr(), cout, cin, 0, st) == 0
    full = torch.empty(B, cout, H, W, device="cuda").bfloat16()
    y = torch.full((B, cout, (H + 1) // 2, (W + 1) // 2), 3.0, device="cuda").bfloat16()
    assert lib.xdna_conv3x3_layout_rows_bf16(xp.data_ptr(), wt.data_ptr(), b.data_ptr(), full.data_ptr(), B, cin,
                                             cout, H, W, 1, st) == 0
    assert lib.xdna_conv3x3_layout_rows_stride2_bf16(xp.data_ptr(), wt.data_ptr(), b.data_ptr(), y.data_ptr(), B,
                                                     cin, cout, H, W, 1, st) == 0
    torch.cuda.synchronize()
    if rows_variant in (1, 4) or (rows_variant == 5 and cout <= 128):
        # no buffer-store epilogue: the stride-2 output took the automatic kernel, whose sums
        # may be ordered otherwise; compare with the automatic stride-1 output
        assert lib.xdna_conv3x3_set_rows_variant(0) == 0
        assert lib.xdna_conv3x3_layout_rows_bf16(xp.data_ptr(), wt.data_ptr(), b.data_ptr(), full.data_ptr(), B, cin,
                                                 cout, H, W, 1, st) == 0
        torch.cuda.synchronize()
    assert torch.equal(y, full[:, :, ::2, ::2])
