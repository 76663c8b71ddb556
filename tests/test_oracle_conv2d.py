"""Pins the oracle's general 2-D convolution (oracle.conv2d_fwd / _dgrad / _wgrad: any
kernel size, stride and padding, dilation 1, groups 1).

1. Brute force: the defining sums, looped element by element on tiny shapes.
2. Library routine: PyTorch CPU float64 conv2d and its autograd gradients (the
   reference's own CPU path for these convolutions) on the style network's and ResNet's
   layer types (9x9 s1, 3x3 s2, 1x1 s1/s2, 7x7 s2), with odd sizes.
3. Adjoint identities, <dy, conv(x)> = <dgrad(dy), x> = <wgrad(x, dy), w>, which a wrong
   index in any one direction breaks.
"""
import numpy as np
import pytest
import torch

import oracle

CASES = [
    # B, Cin, Cout, H, W, KH, KW, sh, sw, ph, pw
    (2, 3, 8, 12, 12, 9, 9, 1, 1, 4, 4),
    (2, 8, 16, 12, 11, 3, 3, 2, 2, 1, 1),
    (2, 16, 8, 7, 9, 1, 1, 1, 1, 0, 0),
    (2, 16, 24, 9, 8, 1, 1, 2, 2, 0, 0),
    (1, 3, 8, 15, 13, 7, 7, 2, 2, 3, 3),
    (1, 4, 5, 6, 7, 3, 2, 1, 3, 1, 0),
]


def _data(case, seed):
    B, Cin, Cout, H, W, KH, KW, sh, sw, ph, pw = case
    rng = np.random.default_rng(seed)
    x = oracle.rng_bf16(rng, (B, Cin, H, W))
    w = oracle.rng_bf16(rng, (Cout, Cin, KH, KW), 0.2)
    b = oracle.rng_bf16(rng, (Cout,), 0.1)
    Ho, Wo = oracle.conv2d_out_size(H, W, KH, KW, sh, sw, ph, pw)
    dy = oracle.rng_bf16(rng, (B, Cout, Ho, Wo))
    return x, w, b, dy


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_against_torch_cpu_float64(case):
    B, Cin, Cout, H, W, KH, KW, sh, sw, ph, pw = case
    x, w, b, dy = _data(case, sum(case))
    xt = torch.from_numpy(oracle.bf16_value(x).astype(np.float64)).requires_grad_()
    wt = torch.from_numpy(oracle.bf16_value(w).astype(np.float64)).requires_grad_()
    bt = torch.from_numpy(oracle.bf16_value(b).astype(np.float64)).requires_grad_()
    y = torch.nn.functional.conv2d(xt, wt, bt, stride=(sh, sw), padding=(ph, pw))
    y.backward(torch.from_numpy(oracle.bf16_value(dy).astype(np.float64)))
    np.testing.assert_allclose(oracle.conv2d_fwd(x, w, b, (sh, sw), (ph, pw)), y.detach().numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.conv2d_dgrad(dy, w, (H, W), (sh, sw), (ph, pw)), xt.grad.numpy(), rtol=1e-12, atol=1e-12)
    gw, gb = oracle.conv2d_wgrad(x, dy, (KH, KW), (sh, sw), (ph, pw))
    np.testing.assert_allclose(gw, wt.grad.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(gb, bt.grad.numpy(), rtol=1e-12, atol=1e-12)


def test_brute_force_tiny():
    case = (1, 2, 3, 5, 4, 3, 2, 2, 1, 1, 0)
    B, Cin, Cout, H, W, KH, KW, sh, sw, ph, pw = case
    x, w, b, dy = _data(case, 3)
    xf, wf, dyf = (oracle.bf16_value(a).astype(np.float64) for a in (x, w, dy))
    Ho, Wo = oracle.conv2d_out_size(H, W, KH, KW, sh, sw, ph, pw)
    y = np.zeros((B, Cout, Ho, Wo))
    dx = np.zeros_like(xf)
    gw = np.zeros_like(wf)
    for bb in range(B):
        for co in range(Cout):
            for oy in range(Ho):
                for ox in range(Wo):
                    for ci in range(Cin):
                        for ky in range(KH):
                            for kx in range(KW):
                                iy, ix = oy * sh - ph + ky, ox * sw - pw + kx
                                if 0 <= iy < H and 0 <= ix < W:
                                    y[bb, co, oy, ox] += wf[co, ci, ky, kx] * xf[bb, ci, iy, ix]
                                    dx[bb, ci, iy, ix] += wf[co, ci, ky, kx] * dyf[bb, co, oy, ox]
                                    gw[co, ci, ky, kx] += dyf[bb, co, oy, ox] * xf[bb, ci, iy, ix]
    np.testing.assert_allclose(oracle.conv2d_fwd(x, w, None, (sh, sw), (ph, pw)), y, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(oracle.conv2d_dgrad(dy, w, (H, W), (sh, sw), (ph, pw)), dx, rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(oracle.conv2d_wgrad(x, dy, (KH, KW), (sh, sw), (ph, pw))[0], gw, rtol=1e-13, atol=1e-13)


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_adjoint_identities(case):
    B, Cin, Cout, H, W, KH, KW, sh, sw, ph, pw = case
    x, w, _, dy = _data(case, 11)
    xf, wf, dyf = (oracle.bf16_value(a).astype(np.float64) for a in (x, w, dy))
    a = np.sum(dyf * oracle.conv2d_fwd(x, w, None, (sh, sw), (ph, pw)))
    b = np.sum(oracle.conv2d_dgrad(dy, w, (H, W), (sh, sw), (ph, pw)) * xf)
    c = np.sum(oracle.conv2d_wgrad(x, dy, (KH, KW), (sh, sw), (ph, pw))[0] * wf)
    assert abs(a - b) <= 1e-9 * max(1.0, abs(a)) and abs(a - c) <= 1e-9 * max(1.0, abs(a))
