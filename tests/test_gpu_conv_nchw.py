"""The small-grid conv reading its NCHW input in place (xdna_conv3x3_nchw_act_bf16) against
the packed path it replaces (xdna_conv3x3_layout_pack_bf16 + xdna_conv3x3_layout_rows_act_bf16
or its stride-2 output form): bit for bit, for both tile heights, split-K over chunks on
small grids, partial 64-channel chunks, partial 64-channel output tiles, bias or none, the
ReLU epilogue and the stride-2 output; and against the double-precision oracle.  Then the
aten path: frozen-weight convs (forward and input gradient) take the NCHW form, trainable
ones keep their packs for the weight gradient."""
import numpy as np
import pytest
import torch

import oracle
import xdna_train
from gpu_util import check_bf16, dev, dev_zeros, host, ptr, stream

pytestmark = pytest.mark.gpu
TIGHT = 1

SHAPES = [
    # B, Cin, Cout, H, W
    (40, 128, 128, 9, 9),    # the style network's residual convs
    (2, 64, 64, 12, 12),
    (1, 128, 64, 9, 9),      # a few workgroups: split-K over the two chunks
    (3, 96, 40, 9, 11),      # partial input chunk, partial output tile
    (4, 32, 64, 36, 36),
    (2, 256, 256, 4, 4),
    (1, 8, 16, 5, 7),
    (6, 64, 128, 18, 18),
]


def _data(B, Cin, Cout, H, W, seed):
    rng = np.random.default_rng(seed)
    bound = np.sqrt(6.0 / (9 * Cin))
    x = oracle.rng_bf16(rng, (B, Cin, H, W))
    w = oracle.bf16_bits(rng.uniform(-bound, bound, (Cout, Cin, 3, 3)).astype(np.float32))
    b = oracle.bf16_bits(rng.uniform(-0.1, 0.1, (Cout,)).astype(np.float32))
    return x, w, b


def _prepared(hip, w, cin, cout):
    n = hip.xdna_conv3x3_prepared_weight_bytes(cin, cout)
    wt = dev_zeros(((n + 1) // 2,))
    assert hip.xdna_conv3x3_prepare_weights_bf16(ptr(dev(w)), ptr(wt), cout, cin, 0, stream()) == 0
    return wt


@pytest.fixture
def variant(hip, request):
    assert hip.xdna_conv3x3_set_rows_variant(request.param) == 0
    yield request.param
    assert hip.xdna_conv3x3_set_rows_variant(0) == 0


@pytest.mark.parametrize("variant", [0, 2, 3], indirect=True, ids=lambda v: f"v{v}")
@pytest.mark.parametrize("act,s2out", [(0, 0), (1, 0), (0, 1)], ids=["plain", "relu", "stride2"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_nchw_matches_packed(hip, shape, act, s2out, variant):
    B, Cin, Cout, H, W = shape
    assert hip.xdna_conv3x3_nchw_small_eligible(B, Cin, Cout, H, W) == 1
    print(f"conv nchw {shape} act {act} s2out {s2out} variant {variant}", flush=True)
    x, w, b = _data(*shape, seed=sum(shape) + 11)
    wt = _prepared(hip, w, Cin, Cout)
    oh, ow = ((H + 1) // 2, (W + 1) // 2) if s2out else (H, W)
    xd, bd = dev(x), dev(b)
    for bias in (bd, None):
        want = dev(np.full((B, Cout, oh, ow), 0x7F7F, np.uint16))
        got = dev(np.full((B, Cout, oh, ow), 0x7F7F, np.uint16))
        n = hip.xdna_conv3x3_layout_packed_bytes(B, Cin, H, W, TIGHT)
        xp = dev_zeros(((n + 1) // 2,))
        assert hip.xdna_conv3x3_layout_pack_bf16(ptr(xd), ptr(xp), B, Cin, H, W, TIGHT, stream()) == 0
        if s2out:
            assert hip.xdna_conv3x3_layout_rows_stride2_bf16(ptr(xp), ptr(wt), ptr(bias), ptr(want), B, Cin, Cout,
                                                             H, W, TIGHT, stream()) == 0
        else:
            assert hip.xdna_conv3x3_layout_rows_act_bf16(ptr(xp), ptr(wt), ptr(bias), ptr(want), B, Cin, Cout, H,
                                                         W, TIGHT, act, stream()) == 0
        assert hip.xdna_conv3x3_nchw_act_bf16(ptr(xd), ptr(wt), ptr(bias), ptr(got), B, Cin, Cout, H, W, act,
                                              s2out, stream()) == 0
        np.testing.assert_array_equal(host(got), host(want))
    # and the oracle (bias, no activation, stride 1)
    if not act and not s2out:
        got = dev_zeros((B, Cout, H, W))
        assert hip.xdna_conv3x3_nchw_act_bf16(ptr(xd), ptr(wt), ptr(bd), ptr(got), B, Cin, Cout, H, W, 0, 0,
                                              stream()) == 0
        check_bf16(host(got), oracle.conv3x3_fwd(x, w, b), what=f"nchw fwd {shape}")


def test_nchw_refuses_what_it_cannot_read(hip):
    """Wider than 36 columns, input channels not a multiple of 8, or a grid the small-grid
    kernel does not take: not eligible, and the entry point refuses with an error."""
    for shape in [(1, 64, 64, 8, 40), (2, 70, 64, 9, 9), (64, 512, 512, 72, 72)]:
        B, Cin, Cout, H, W = shape
        assert hip.xdna_conv3x3_nchw_small_eligible(B, Cin, Cout, H, W) == 0
        assert hip.xdna_conv3x3_nchw_act_bf16(1, 1, None, 1, B, Cin, Cout, H, W, 0, 0, stream()) == -1


def _calls(name):
    return xdna_train.mapped_cpu_stats().get(name, {}).get("calls", 0)


@pytest.mark.parametrize("frozen", [True, False])
def test_aten_route(frozen):
    """Through aten: a frozen 3x3 conv's forward and input gradient read their NCHW inputs
    (no pack); a trainable one packs x (kept for its weight gradient) and dY.  Results
    against the oracle."""
    X = torch.device("xdna")
    torch.manual_seed(5)
    conv = torch.nn.Conv2d(64, 64, 3, padding=1).bfloat16().to(X)
    conv.weight.requires_grad_(not frozen)
    conv.bias.requires_grad_(not frozen)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(8, 64, 9, 9, generator=g).bfloat16()
    dy = torch.randn(8, 64, 9, 9, generator=g).bfloat16()
    xd = x.to(X).requires_grad_()
    xdna_train.synchronize()
    xdna_train.reset_mapped_cpu_stats()
    y = conv(xd)
    y.backward(dy.to(X))
    xdna_train.synchronize()
    assert _calls("hip_conv3x3.nchw") == (2 if frozen else 0)
    bits = lambda t: t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    xb, wb, bb, db = bits(x), bits(conv.weight), bits(conv.bias), bits(dy)
    check_bf16(bits(y), oracle.conv3x3_fwd(xb, wb, bb), what="aten fwd")
    check_bf16(bits(xd.grad), oracle.conv3x3_dgrad(db, wb), what="aten dgrad")
