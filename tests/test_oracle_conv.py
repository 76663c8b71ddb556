"""Pins the oracle's direct convolutions (oracle_conv3x3_fwd / _dgrad / _wgrad).

* brute force in pure Python on tiny shapes (independent loop order and indexing);
* PyTorch's CPU float64 conv2d and its input/weight gradients (a library routine);
* closed forms: zero input -> bias, centre-tap identity kernel -> copy, a one-tap
  kernel -> translation with zero fill;
* adjoint identities <dy, conv(x, w)> = <dgrad(dy, w), x> = <wgrad(x, dy), w>, which
  a transposed or flipped index in dgrad/wgrad breaks.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle


def _bf(rng, shape, scale=1.0):
    return oracle.rng_bf16(rng, shape, scale)


def _val(bits):
    return oracle.bf16_value(bits).astype(np.float64)


def _brute_fwd(x, w, b):
    B, Cin, H, W = x.shape
    Cout = w.shape[0]
    y = np.zeros((B, Cout, H, W))
    for n in range(B):
        for co in range(Cout):
            for i in range(H):
                for j in range(W):
                    s = b[co] if b is not None else 0.0
                    for ci in range(Cin):
                        for dy in range(3):
                            for dx in range(3):
                                ii, jj = i + dy - 1, j + dx - 1
                                if 0 <= ii < H and 0 <= jj < W:
                                    s += x[n, ci, ii, jj] * w[co, ci, dy, dx]
                    y[n, co, i, j] = s
    return y


def test_brute_force_tiny():
    rng = np.random.default_rng(0)
    B, Cin, Cout, H, W = 2, 3, 2, 4, 5
    x, w, b = _bf(rng, (B, Cin, H, W)), _bf(rng, (Cout, Cin, 3, 3)), _bf(rng, (Cout,))
    ref = _brute_fwd(_val(x), _val(w), _val(b))
    np.testing.assert_allclose(oracle.conv3x3_fwd(x, w, b), ref, rtol=1e-12, atol=1e-12)
    # dgrad / wgrad by brute-force differentiation of the (linear) forward
    dy = _bf(rng, (B, Cout, H, W))
    dx_ref = np.zeros((B, Cin, H, W))
    for idx in np.ndindex(B, Cin, H, W):
        e = np.zeros((B, Cin, H, W))
        e[idx] = 1.0
        dx_ref[idx] = np.sum(_brute_fwd(e, _val(w), None) * _val(dy))
    np.testing.assert_allclose(oracle.conv3x3_dgrad(dy, w), dx_ref, rtol=1e-12, atol=1e-12)
    gw_ref = np.zeros((Cout, Cin, 3, 3))
    for idx in np.ndindex(Cout, Cin, 3, 3):
        e = np.zeros((Cout, Cin, 3, 3))
        e[idx] = 1.0
        gw_ref[idx] = np.sum(_brute_fwd(_val(x), e, None) * _val(dy))
    gw, gb = oracle.conv3x3_wgrad(x, dy)
    np.testing.assert_allclose(gw, gw_ref, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(gb, _val(dy).sum(axis=(0, 2, 3)), rtol=1e-12)


@pytest.mark.parametrize("B,Cin,Cout,H,W", [(2, 5, 7, 9, 11), (1, 64, 32, 6, 40), (3, 3, 8, 13, 1)])
def test_against_torch_float64(B, Cin, Cout, H, W):
    rng = np.random.default_rng(B * 100 + Cin)
    x, w, b, dy = (_bf(rng, (B, Cin, H, W)), _bf(rng, (Cout, Cin, 3, 3), 0.2), _bf(rng, (Cout,)),
                   _bf(rng, (B, Cout, H, W)))
    tx, tw, tb, tdy = (torch.from_numpy(_val(a)) for a in (x, w, b, dy))
    y = F.conv2d(tx, tw, tb, padding=1).numpy()
    np.testing.assert_allclose(oracle.conv3x3_fwd(x, w, b), y, rtol=1e-10, atol=1e-10)
    dx = torch.nn.grad.conv2d_input(tx.shape, tw, tdy, padding=1).numpy()
    np.testing.assert_allclose(oracle.conv3x3_dgrad(dy, w), dx, rtol=1e-10, atol=1e-10)
    gw = torch.nn.grad.conv2d_weight(tx, tw.shape, tdy, padding=1).numpy()
    ogw, ogb = oracle.conv3x3_wgrad(x, dy)
    np.testing.assert_allclose(ogw, gw, rtol=1e-10, atol=1e-9)
    np.testing.assert_allclose(ogb, tdy.sum(dim=(0, 2, 3)).numpy(), rtol=1e-12, atol=1e-12)


def test_closed_forms():
    rng = np.random.default_rng(1)
    B, C, H, W = 2, 4, 5, 6
    b = _bf(rng, (C,))
    zero = np.zeros((B, C, H, W), np.uint16)
    w = _bf(rng, (C, C, 3, 3))
    y = oracle.conv3x3_fwd(zero, w, b)
    np.testing.assert_array_equal(y, np.broadcast_to(_val(b)[None, :, None, None], y.shape))
    x = _bf(rng, (B, C, H, W))
    ident = np.zeros((C, C, 3, 3), np.float32)
    for c in range(C):
        ident[c, c, 1, 1] = 1.0
    np.testing.assert_array_equal(oracle.conv3x3_fwd(x, oracle.bf16_bits(ident)), _val(x))
    # tap (dy, dx) = (0, 2): y[i][j] = x[i-1][j+1], zero outside
    shift = np.zeros((C, C, 3, 3), np.float32)
    for c in range(C):
        shift[c, c, 0, 2] = 1.0
    ys = oracle.conv3x3_fwd(x, oracle.bf16_bits(shift))
    exp = np.zeros_like(ys)
    exp[:, :, 1:, :-1] = _val(x)[:, :, :-1, 1:]
    np.testing.assert_array_equal(ys, exp)


@pytest.mark.parametrize("B,Cin,Cout,H,W", [(2, 6, 5, 7, 8), (1, 70, 9, 4, 37)])
def test_adjoint_identities(B, Cin, Cout, H, W):
    rng = np.random.default_rng(11)
    x, w, dy = _bf(rng, (B, Cin, H, W)), _bf(rng, (Cout, Cin, 3, 3)), _bf(rng, (B, Cout, H, W))
    a = np.sum(_val(dy) * oracle.conv3x3_fwd(x, w))
    b_ = np.sum(oracle.conv3x3_dgrad(dy, w) * _val(x))
    gw, _ = oracle.conv3x3_wgrad(x, dy)
    c = np.sum(gw * _val(w))
    assert abs(a - b_) <= 1e-9 * max(1.0, abs(a))
    assert abs(a - c) <= 1e-9 * max(1.0, abs(a))


def test_linearity():
    rng = np.random.default_rng(4)
    x1 = _bf(rng, (1, 3, 6, 6))
    x2 = _bf(rng, (1, 3, 6, 6))
    w = _bf(rng, (2, 3, 3, 3))
    y12 = oracle.conv3x3_fwd(x1, w) + oracle.conv3x3_fwd(x2, w)
    # conv of x1 + x2 through the float64 route: split into two exactly representable halves
    np.testing.assert_allclose(_brute_fwd(_val(x1) + _val(x2), _val(w), None), y12, rtol=1e-12, atol=1e-12)
