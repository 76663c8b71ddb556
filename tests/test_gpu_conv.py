"""HIP 3x3 conv forward / dgrad / wgrad (+ bias grad) vs the double-precision oracle.

Bar: every output within 2 bf16 ulp of the exact sum of the bf16
operands (with a floor at ulp(max|ref| * 2^-8) for outputs that cancel to ~0) and
relative L2 <= 1e-2.  Shapes cover ragged channel counts (partial 64-chunks, partial
128-blocks), one and several 2048-row groups, tiny channel counts (RGB-like), width
strips (W > 36: S = 2, 3) and the C1 conv at B = 2.  Forward and dgrad run through each
rows-kernel variant (main kernel; small-grid kernel with 64 / 128-row tiles, split-K over
chunks on small grids; wide kernels with 256-channel tiles in eight- and four-wave forms;
four-wave kernels with 128- and 64-channel tiles).  wgrad is also checked for run-to-run bit equality (its split-K
reduction is fixed-order).
"""
import numpy as np
import pytest

import layout_util
import oracle
from gpu_util import check_bf16, dev, dev_zeros, host, ptr, stream

pytestmark = pytest.mark.gpu

SHAPES = [
    # B, Cin, Cout, H, W
    (2, 64, 64, 12, 12),
    (3, 70, 130, 9, 11),
    (2, 3, 32, 7, 5),
    (1, 64, 64, 8, 40),
    (2, 128, 128, 36, 36),
    (4, 64, 64, 36, 36),
    (1, 128, 256, 18, 72),
    (2, 256, 64, 5, 37),
    (1, 1, 1, 1, 1),
    (1, 64, 384, 6, 40),    # 384 output channels: a partial 256-channel tile
    (5, 96, 260, 24, 24),   # two groups, two chunks, a 4-channel second 256-channel tile
]


def _data(B, Cin, Cout, H, W, seed):
    rng = np.random.default_rng(seed)
    bound = np.sqrt(6.0 / (9 * Cin))
    x = oracle.rng_bf16(rng, (B, Cin, H, W))
    w = oracle.bf16_bits(rng.uniform(-bound, bound, (Cout, Cin, 3, 3)).astype(np.float32))
    b = oracle.bf16_bits(rng.uniform(-0.1, 0.1, (Cout,)).astype(np.float32))
    dy = oracle.rng_bf16(rng, (B, Cout, H, W))
    return x, w, b, dy


def _ws(nbytes):
    return dev_zeros((max(1, (nbytes + 1) // 2),))


# rows-kernel variants (xdna_conv3x3_set_rows_variant): main kernel, small-grid kernel
# with 64- and 128-row tiles (split-K over chunks where the grid is small), wide kernel
# with eight and with four waves (256-channel tiles, for cout > 128; the main kernel
# otherwise), four-wave kernels with 128 x 256, 128 x 512 and 64 x 512 tiles, 64 x 256
# tiles two per CU, and the 16x16x32 MFMA forms of the 128 x 512 and 64 x 256 tiles
VARIANTS = [1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11]


@pytest.fixture
def variant(hip, request):
    assert hip.xdna_conv3x3_set_rows_variant(request.param) == 0
    yield request.param
    assert hip.xdna_conv3x3_set_rows_variant(0) == 0


@pytest.mark.parametrize("variant", VARIANTS, indirect=True, ids=lambda v: f"v{v}")
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_forward(hip, shape, variant):
    B, Cin, Cout, H, W = shape
    print(f"conv fwd {shape} variant {variant}", flush=True)
    x, w, b, _ = _data(*shape, seed=sum(shape))
    ref = oracle.conv3x3_fwd(x, w, b)
    ws_bytes = hip.xdna_conv3x3_fwd_workspace_bytes(B, Cin, Cout, H, W)
    ws = _ws(ws_bytes)
    y = dev_zeros((B, Cout, H, W))
    assert hip.xdna_conv3x3_fwd_bf16(ptr(dev(x)), ptr(dev(w)), ptr(dev(b)), ptr(y), B, Cin, Cout, H, W,
                                     ptr(ws), ws_bytes, stream()) == 0
    check_bf16(host(y), ref, what=f"fwd {shape}")
    # without bias
    y2 = dev_zeros((B, Cout, H, W))
    assert hip.xdna_conv3x3_fwd_bf16(ptr(dev(x)), ptr(dev(w)), None, ptr(y2), B, Cin, Cout, H, W,
                                     ptr(ws), ws_bytes, stream()) == 0
    check_bf16(host(y2), oracle.conv3x3_fwd(x, w), what=f"fwd nobias {shape}")


@pytest.mark.parametrize("variant", VARIANTS, indirect=True, ids=lambda v: f"v{v}")
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_dgrad(hip, shape, variant):
    B, Cin, Cout, H, W = shape
    print(f"conv dgrad {shape} variant {variant}", flush=True)
    _, w, _, dy = _data(*shape, seed=sum(shape) + 1)
    ref = oracle.conv3x3_dgrad(dy, w)
    ws_bytes = hip.xdna_conv3x3_dgrad_workspace_bytes(B, Cin, Cout, H, W)
    ws = _ws(ws_bytes)
    dx = dev_zeros((B, Cin, H, W))
    assert hip.xdna_conv3x3_dgrad_bf16(ptr(dev(dy)), ptr(dev(w)), ptr(dx), B, Cin, Cout, H, W, ptr(ws),
                                       ws_bytes, stream()) == 0
    check_bf16(host(dx), ref, what=f"dgrad {shape}")


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_wgrad(hip, shape):
    B, Cin, Cout, H, W = shape
    print(f"conv wgrad {shape}", flush=True)
    x, _, _, dy = _data(*shape, seed=sum(shape) + 2)
    ref_w, ref_b = oracle.conv3x3_wgrad(x, dy)
    ws_bytes = hip.xdna_conv3x3_wgrad_workspace_bytes(B, Cin, Cout, H, W)
    ws = _ws(ws_bytes)
    gw = dev_zeros((Cout, Cin, 3, 3))
    gb = dev_zeros((Cout,))
    dx_, ddy = dev(x), dev(dy)
    assert hip.xdna_conv3x3_wgrad_bf16(ptr(dx_), ptr(ddy), ptr(gw), ptr(gb), B, Cin, Cout, H, W, ptr(ws),
                                       ws_bytes, stream()) == 0
    got_w, got_b = host(gw), host(gb)
    check_bf16(got_w, ref_w, what=f"wgrad {shape}")
    check_bf16(got_b, ref_b, what=f"bias grad {shape}")
    # deterministic: a second call gives the same bits
    gw2 = dev_zeros((Cout, Cin, 3, 3))
    assert hip.xdna_conv3x3_wgrad_bf16(ptr(dx_), ptr(ddy), ptr(gw2), None, B, Cin, Cout, H, W, ptr(ws),
                                       ws_bytes, stream()) == 0
    np.testing.assert_array_equal(host(gw2), got_w)
    # standalone bias gradient
    gb2 = dev_zeros((Cout,))
    assert hip.xdna_conv3x3_bias_grad_bf16(ptr(ddy), ptr(gb2), B, Cout, H, W, stream()) == 0
    check_bf16(host(gb2), ref_b, what=f"bias grad kernel {shape}")


# shapes whose layouts differ (W > 36), one where they agree, and one past the LDS tile
LAYOUT_SHAPES = [(1, 64, 64, 8, 40), (1, 128, 256, 18, 72), (2, 256, 64, 5, 37), (1, 64, 384, 6, 40),
                 (1, 32, 48, 5, 110), (1, 16, 24, 3, 300), (2, 64, 64, 12, 12)]


def _pack(hip, bits, layout):
    """bits packed on the device in `layout` into a buffer pre-filled with a non-zero pattern."""
    B, C, H, W = bits.shape
    n = hip.xdna_conv3x3_layout_packed_bytes(B, C, H, W, layout)
    assert n > 0
    buf = dev(np.full((n // 2,), 0xBEEF, np.uint16))
    assert hip.xdna_conv3x3_layout_pack_bf16(ptr(dev(bits)), ptr(buf), B, C, H, W, layout, stream()) == 0
    return buf


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("shape", LAYOUT_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_layout_pack(hip, shape, layout):
    """Both row layouts written whole (zeros included) and bit-exact against the host
    construction (itself pinned to the oracle's reference pack on the CPU)."""
    B, Cin, _, H, W = shape
    print(f"layout pack {shape} layout {layout}", flush=True)
    x = _data(*shape, seed=sum(shape) + 5)[0]
    got = host(_pack(hip, x, layout)).reshape(-1)
    np.testing.assert_array_equal(got, layout_util.pack_expected(x, layout).reshape(-1))
    assert hip.xdna_conv3x3_layout_packed_bytes(B, Cin, H, W, 2) == 0


@pytest.mark.parametrize("variant", VARIANTS, indirect=True, ids=lambda v: f"v{v}")
@pytest.mark.parametrize("shape", LAYOUT_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_forward_tight_layout(hip, shape, variant):
    """The rows kernels on the tight layout (every variant) vs the oracle."""
    B, Cin, Cout, H, W = shape
    print(f"conv fwd tight {shape} variant {variant}", flush=True)
    x, w, b, _ = _data(*shape, seed=sum(shape) + 6)
    xp = _pack(hip, x, 1)
    wt = _ws(hip.xdna_conv3x3_prepared_weight_bytes(Cin, Cout))
    assert hip.xdna_conv3x3_prepare_weights_bf16(ptr(dev(w)), ptr(wt), Cout, Cin, 0, stream()) == 0
    y = dev_zeros((B, Cout, H, W))
    assert hip.xdna_conv3x3_layout_rows_bf16(ptr(xp), ptr(wt), ptr(dev(b)), ptr(y), B, Cin, Cout, H, W, 1,
                                             stream()) == 0
    check_bf16(host(y), oracle.conv3x3_fwd(x, w, b), what=f"fwd tight {shape}")


@pytest.fixture(params=[(1, 128, 0), (1, 64, 0), (2, 64, 0), (2, 64, 64), (2, 64, 128)],
                ids=lambda p: f"form{p[0]}-kt{p[1]}-tile{p[2]}")
def wgrad_kt(hip, request):
    """Kernel form of the rows weight gradient (1: register-staged k-tiles of 128 or 64
    rows, 2: 64-row k-tiles loaded straight into LDS, its output-channel tile by layer (0),
    or forced to 64 (four waves) or 128 (eight waves)) and its k-tile rows."""
    form, kt, tile = request.param
    assert hip.xdna_conv3x3_set_wgrad_rows_kernel(form) == 0
    assert hip.xdna_conv3x3_set_wgrad_rows_kt(kt) == 0
    assert hip.xdna_conv3x3_set_wgrad_tile(tile) == 0
    yield kt
    assert hip.xdna_conv3x3_set_wgrad_tile(0) == 0
    assert hip.xdna_conv3x3_set_wgrad_rows_kt(0) == 0
    assert hip.xdna_conv3x3_set_wgrad_rows_kernel(0) == 0


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("shape", SHAPES + LAYOUT_SHAPES[4:6], ids=lambda s: "x".join(map(str, s)))
def test_wgrad_rows(hip, shape, layout, wgrad_kt):
    """Weight gradient from the packed row layouts (x and dY packed as the forward and
    input-gradient convs pack them), with 128- and 64-row k-tiles, vs the oracle; run-to-run
    bit equality."""
    B, Cin, Cout, H, W = shape
    print(f"conv wgrad rows {shape} layout {layout} kt {wgrad_kt}", flush=True)
    x, _, _, dy = _data(*shape, seed=sum(shape) + 3)
    ref_w, ref_b = oracle.conv3x3_wgrad(x, dy)
    xp = _pack(hip, x, layout)
    dp = _pack(hip, dy, layout)
    ws_bytes = hip.xdna_conv3x3_wgrad_rows_workspace_bytes(B, Cin, Cout, H, W, layout)
    ws = _ws(ws_bytes)
    gw = dev_zeros((Cout, Cin, 3, 3))
    gb = dev_zeros((Cout,))
    assert hip.xdna_conv3x3_wgrad_rows_bf16(ptr(xp), ptr(dp), ptr(gw), ptr(gb), B, Cin, Cout, H, W, layout,
                                            ptr(ws), ws_bytes, stream()) == 0
    got_w = host(gw)
    check_bf16(got_w, ref_w, what=f"wgrad rows {shape}")
    check_bf16(host(gb), ref_b, what=f"bias grad rows {shape}")
    gw2 = dev_zeros((Cout, Cin, 3, 3))
    assert hip.xdna_conv3x3_wgrad_rows_bf16(ptr(xp), ptr(dp), ptr(gw2), None, B, Cin, Cout, H, W, layout,
                                            ptr(ws), ws_bytes, stream()) == 0
    np.testing.assert_array_equal(host(gw2), got_w)
    assert hip.xdna_conv3x3_wgrad_rows_bf16(ptr(xp), ptr(dp), ptr(gw2), None, B, Cin, Cout, H, W, layout,
                                            ptr(ws), ws_bytes - 1, stream()) == -1


def test_wgrad_rows_kt_setter_rejects(hip):
    assert hip.xdna_conv3x3_set_wgrad_rows_kt(96) == -1
    assert hip.xdna_conv3x3_set_wgrad_rows_kt(0) == 0
    assert hip.xdna_conv3x3_set_wgrad_rows_kernel(3) == -1
    assert hip.xdna_conv3x3_set_wgrad_rows_kernel(0) == 0
    assert hip.xdna_conv3x3_set_wgrad_tile(96) == -1
    assert hip.xdna_conv3x3_set_wgrad_tile(0) == 0


def test_workspace_too_small_is_an_error(hip):
    B, C, H, W = 1, 8, 4, 4
    ws = _ws(64)
    y = dev_zeros((B, C, H, W))
    x = dev_zeros((B, C, H, W))
    w = dev_zeros((C, C, 3, 3))
    rc = hip.xdna_conv3x3_fwd_bf16(ptr(x), ptr(w), None, ptr(y), B, C, C, H, W, ptr(ws), 64, stream())
    assert rc == -1


def _prepared_expected(w, dgrad):
    """The prepared form on the host: rows = the conv's output channels padded to 128 (or a
    multiple of 256 beyond 128), k = (64-channel chunk, tap, channel); the input-gradient
    form is that of w'[ci][co][t] = w[co][ci][8 - t]."""
    Cout, Cin = w.shape[:2]
    wf = w.reshape(Cout, Cin, 9)
    if dgrad:
        wf = wf[:, :, ::-1].transpose(1, 0, 2)
    rows, cols = wf.shape[:2]
    co_pad = 128 if rows <= 128 else -(-rows // 256) * 256
    chunks = -(-cols // 64)
    tmp = np.zeros((co_pad, chunks * 64, 9), np.uint16)
    tmp[:rows, :cols] = wf
    return tmp.reshape(co_pad, chunks, 64, 9).transpose(0, 1, 3, 2).reshape(-1)


@pytest.mark.parametrize("tile", [0, 8, 32])
@pytest.mark.parametrize("cin,cout", [(3, 64), (64, 64), (128, 128), (256, 512), (512, 256), (100, 36), (36, 300),
                                      (8, 3), (520, 130)])
def test_prepared_weights_bit_exact(hip, cin, cout, tile):
    """Both prepared forms, from the single-form and the two-form entry points, bit-exact
    against the host construction (every padded element zero), with the preparation's
    output-channel tile chosen by size (0) or forced to 8 or 32."""
    assert hip.xdna_conv3x3_set_prep_tile(tile) == 0
    try:
        _check_prepared(hip, cin, cout)
    finally:
        hip.xdna_conv3x3_set_prep_tile(0)


def _check_prepared(hip, cin, cout):
    rng = np.random.default_rng(cin * 1000 + cout)
    w = oracle.rng_bf16(rng, (cout, cin, 3, 3))
    wd = dev(w)
    nf = hip.xdna_conv3x3_prepared_weight_bytes(cin, cout)
    nd = hip.xdna_conv3x3_prepared_weight_bytes(cout, cin)
    for dgrad, n in ((0, nf), (1, nd)):
        out = dev_zeros((n // 2,)) - 1  # every element must be written
        assert hip.xdna_conv3x3_prepare_weights_bf16(ptr(wd), ptr(out), cout, cin, dgrad, stream()) == 0
        exp = _prepared_expected(w, dgrad)
        np.testing.assert_array_equal(host(out)[:exp.size], exp, err_msg=f"form {dgrad}")
    of, od = dev_zeros((nf // 2,)) - 1, dev_zeros((nd // 2,)) - 1
    assert hip.xdna_conv3x3_prepare_weights_both_bf16(ptr(wd), ptr(of), ptr(od), cout, cin, stream()) == 0
    np.testing.assert_array_equal(host(of)[:_prepared_expected(w, 0).size], _prepared_expected(w, 0))
    np.testing.assert_array_equal(host(od)[:_prepared_expected(w, 1).size], _prepared_expected(w, 1))
