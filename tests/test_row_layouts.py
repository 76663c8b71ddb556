"""The host construction of the packed row layouts (tests/layout_util.py) on the CPU:
layout 0 against the oracle's restatement of the reference's conv3x3w pack
(conv_pack.cpp:632-743), and both layouts as conv layouts: the rows-kernel recipe (output
row p sums grid rows p + dy*wp + dx) over each layout gives the float64 oracle conv.  The
GPU tests compare the device packs of both layouts with this construction."""
import numpy as np
import pytest

import oracle
import layout_util as lu

SHAPES = [(2, 5, 4, 7), (1, 70, 3, 36), (2, 3, 5, 37), (1, 64, 3, 40), (1, 9, 4, 72), (2, 4, 2, 73),
          (1, 3, 2, 110), (1, 2, 2, 300)]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_reference_layout_matches_oracle_pack(shape):
    B, C, H, W = shape
    x = oracle.rng_bf16(np.random.default_rng(sum(shape)), shape)
    assert lu.strip_params(W, 0)[:2] == oracle.strip_geometry(W)
    S, So, Wg, wp, m_total, groups = oracle.geometry(B, H, W)
    assert lu.geometry(B, H, W, 0)[:4] == (S, So, Wg, wp)
    np.testing.assert_array_equal(lu.pack_expected(x, 0), oracle.pack(x, B, C, H, W))


@pytest.mark.parametrize("W", list(range(1, 40)) + [70, 71, 72, 73, 107, 108, 109, 256, 300, 1000])
def test_tight_strip_geometry(W):
    S, So, Wg, wp, lead, first = lu.strip_params(W, 1)
    if W <= 36:
        assert lu.strip_params(W, 1) == lu.strip_params(W, 0)
        return
    assert S * So >= W and (S - 1) * So < W and So <= 36
    assert wp == Wg == So + 2 and lead == 0 and first == 0
    # the window of the kernels' groups: 2048 + 2*wp + 2 rows at most
    assert 2 * wp + 2 <= lu.GROUP_ROWS - lu.GROUP_OUT
    # never more strips than the reference layout's
    assert S <= lu.strip_params(W, 0)[0]


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("shape", [(2, 3, 4, 5, 7), (1, 5, 3, 4, 40), (2, 4, 2, 3, 73), (1, 2, 3, 2, 110)],
                         ids=lambda s: "x".join(map(str, s)))
def test_layouts_compute_the_conv(shape, layout):
    B, Cin, Cout, H, W = shape
    rng = np.random.default_rng(sum(shape) + layout)
    x = oracle.rng_bf16(rng, (B, Cin, H, W))
    w = oracle.rng_bf16(rng, (Cout, Cin, 3, 3))
    ref = oracle.conv3x3_fwd(x, w)
    got = lu.conv_by_rows(oracle.bf16_value(x).astype(np.float64), oracle.bf16_value(w).astype(np.float64), layout)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
