"""HIP general 2-D convolution (xdna_conv2d_*: any kernel, stride, padding) vs the
float64 oracle, to the conv bar: every output within 2 bf16 ulp of the exact sum of the
bf16 operands (floor at ulp(max|ref| * 2^-8)) and relative L2 <= 1e-2.

Shapes: the style network's 9x9 input / output layers and stride-2 encoder convs,
ResNet's 7x7 stride-2 stem and 1x1 stride-2 downsampling, non-square kernels and
strides, odd sizes, channel counts that leave partial 32 / 64 / 128-row tiles, and a
pixel count beyond one 128-column tile row.  The weight gradient is checked for
run-to-run bit equality (fixed-order split reduction).  Forward and input gradient run
in both kernel forms: automatic (the direct form at stride 1 with <= 32 output and >= 16
input channels of the direction, up to the widest padded row it stages) and the gather
GEMM alone.
"""
import numpy as np
import pytest

import oracle
from gpu_util import check_bf16, dev, dev_zeros, host, ptr, stream

pytestmark = pytest.mark.gpu

CASES = [
    # B, Cin, Cout, H, W, KH, KW, sh, sw, ph, pw
    (4, 3, 32, 36, 36, 9, 9, 1, 1, 4, 4),     # style: 9x9 3->32
    (4, 32, 3, 36, 36, 9, 9, 1, 1, 4, 4),     # style: 9x9 32->3
    (4, 32, 64, 36, 36, 3, 3, 2, 2, 1, 1),    # style: 3x3 s2 32->64
    (4, 64, 128, 18, 18, 3, 3, 2, 2, 1, 1),   # style: 3x3 s2 64->128
    (2, 3, 64, 32, 32, 7, 7, 2, 2, 3, 3),     # ResNet stem
    (4, 64, 128, 16, 16, 1, 1, 2, 2, 0, 0),   # ResNet 1x1 s2 downsample
    (3, 40, 70, 9, 11, 1, 1, 1, 1, 0, 0),     # 1x1, partial tiles
    (2, 5, 130, 7, 9, 3, 2, 1, 3, 1, 0),      # non-square kernel and stride
    (1, 1, 1, 1, 1, 1, 1, 1, 1, 0, 0),
    (2, 70, 20, 13, 17, 5, 3, 1, 1, 2, 1),    # direct form: 3 channel chunks (partial), 5x3
    (3, 16, 32, 40, 50, 3, 3, 1, 1, 0, 0),    # direct form: no padding, 7 grid blocks
    (2, 16, 5, 30, 90, 7, 7, 1, 1, 3, 3),     # direct form: wide row (12 grid blocks, 95 KB LDS)
    (2, 6, 4, 20, 200, 3, 3, 1, 1, 1, 1),     # too wide for the direct form: gather GEMM
]


@pytest.fixture(params=[0, 1], ids=["auto", "gather"])
def cvar(request, hip):
    assert hip.xdna_conv2d_set_variant(request.param) == 0
    yield request.param
    hip.xdna_conv2d_set_variant(0)


def _data(case, seed):
    B, Cin, Cout, H, W, KH, KW, sh, sw, ph, pw = case
    rng = np.random.default_rng(seed)
    bound = np.sqrt(6.0 / (Cin * KH * KW))
    x = oracle.rng_bf16(rng, (B, Cin, H, W))
    w = oracle.bf16_bits(rng.uniform(-bound, bound, (Cout, Cin, KH, KW)).astype(np.float32))
    b = oracle.bf16_bits(rng.uniform(-0.1, 0.1, (Cout,)).astype(np.float32))
    Ho, Wo = oracle.conv2d_out_size(H, W, KH, KW, sh, sw, ph, pw)
    dy = oracle.rng_bf16(rng, (B, Cout, Ho, Wo))
    return x, w, b, dy, Ho, Wo


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_forward(hip, case, cvar):
    B, Cin, Cout, H, W, KH, KW, sh, sw, ph, pw = case
    print(f"conv2d fwd {case} variant {cvar}", flush=True)
    x, w, b, _, Ho, Wo = _data(case, sum(case))
    y = dev_zeros((B, Cout, Ho, Wo))
    assert hip.xdna_conv2d_fwd_bf16(ptr(dev(x)), ptr(dev(w)), ptr(dev(b)), ptr(y), B, Cin, Cout, H, W, KH, KW,
                                    sh, sw, ph, pw, stream()) == 0
    check_bf16(host(y), oracle.conv2d_fwd(x, w, b, (sh, sw), (ph, pw)), what=f"fwd {case}")
    y2 = dev_zeros((B, Cout, Ho, Wo))
    assert hip.xdna_conv2d_fwd_bf16(ptr(dev(x)), ptr(dev(w)), None, ptr(y2), B, Cin, Cout, H, W, KH, KW,
                                    sh, sw, ph, pw, stream()) == 0
    check_bf16(host(y2), oracle.conv2d_fwd(x, w, None, (sh, sw), (ph, pw)), what=f"fwd nobias {case}")


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_dgrad(hip, case, cvar):
    B, Cin, Cout, H, W, KH, KW, sh, sw, ph, pw = case
    print(f"conv2d dgrad {case} variant {cvar}", flush=True)
    _, w, _, dy, Ho, Wo = _data(case, sum(case) + 1)
    dx = dev_zeros((B, Cin, H, W))
    assert hip.xdna_conv2d_dgrad_bf16(ptr(dev(dy)), ptr(dev(w)), ptr(dx), B, Cin, Cout, H, W, KH, KW, sh, sw,
                                      ph, pw, stream()) == 0
    check_bf16(host(dx), oracle.conv2d_dgrad(dy, w, (H, W), (sh, sw), (ph, pw)), what=f"dgrad {case}")


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_wgrad(hip, case):
    B, Cin, Cout, H, W, KH, KW, sh, sw, ph, pw = case
    print(f"conv2d wgrad {case}", flush=True)
    x, _, _, dy, Ho, Wo = _data(case, sum(case) + 2)
    gw = dev_zeros((Cout, Cin, KH, KW))
    gb = dev_zeros((Cout,))
    dx_, ddy = dev(x), dev(dy)
    assert hip.xdna_conv2d_wgrad_bf16(ptr(dx_), ptr(ddy), ptr(gw), ptr(gb), B, Cin, Cout, H, W, KH, KW, sh, sw,
                                      ph, pw, stream()) == 0
    ref_w, ref_b = oracle.conv2d_wgrad(x, dy, (KH, KW), (sh, sw), (ph, pw))
    got = host(gw)
    check_bf16(got, ref_w, what=f"wgrad {case}")
    check_bf16(host(gb), ref_b, what=f"bias grad {case}")
    gw2 = dev_zeros((Cout, Cin, KH, KW))
    assert hip.xdna_conv2d_wgrad_bf16(ptr(dx_), ptr(ddy), ptr(gw2), None, B, Cin, Cout, H, W, KH, KW, sh, sw,
                                      ph, pw, stream()) == 0
    np.testing.assert_array_equal(host(gw2), got)


def test_invalid_shapes(hip):
    y = dev_zeros((1,))
    assert hip.xdna_conv2d_fwd_bf16(ptr(y), ptr(y), None, ptr(y), 1, 1, 1, 2, 2, 5, 5, 1, 1, 0, 0, stream()) == -1
    assert "kernel larger" in hip.xdna_hip_last_error().decode()
    assert hip.xdna_conv2d_fwd_bf16(ptr(y), ptr(y), None, ptr(y), 1, 1, 1, 2, 2, 1, 1, 0, 1, 0, 0, stream()) == -1
