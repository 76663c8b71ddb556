"""The BFP16 emulation of the reference NPU's conv arithmetic on the GPU
(xdna_bfp16_quantize8_bf16, xdna_conv3x3_layout_rows_bfp16_emul_bf16, and the aten route
behind xdna_train.set_bfp16_emulation), against the oracle's restatement
(oracle_bfp16_quantize8 / oracle_conv3x3_bfp16_emul, pinned in
tests/test_oracle_bfp16_emul.py against the codec and the reference gate's formulation)
and against the GPU's own BFP16 codec kernels.

Bars: the quantization bit for bit (every bf16 pattern included); the emulated conv bit
for bit on all but 1e-4 of the outputs and within one bf16 ulp on those (the GPU sums a
chunk's 64 products in fp32, the oracle in double: with BFP16 operands the fp32 sums are
exact unless the blocks' exponents spread over more than ~8 bits, which rounding can then
move by one ulp); weight gradients exact, as in the reference (its gate's default).
"""
import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
import xdna_train
from gpu_util import check_bf16, dev, dev_zeros, host, ptr, stream

pytestmark = pytest.mark.gpu
X = torch.device("xdna")
TIGHT = 1


def _agree(got, want, what, frac=1e-4):
    g = oracle.bf16_value(got).astype(np.float64)
    w = oracle.bf16_value(want).astype(np.float64)
    same = (got == want) | (np.isnan(g) & np.isnan(w))
    n_diff = int(np.sum(~same))
    print(f"{what}: {n_diff} of {got.size} outputs differ from the oracle", flush=True)
    assert n_diff <= frac * got.size, f"{what}: {n_diff} outputs differ"
    if n_diff:
        assert np.all(np.abs(g - w)[~same] <= oracle.bf16_ulp(w)[~same]), f"{what}: a difference beyond one ulp"


def test_quantization_kernel_matches_oracle(hip):
    rng = np.random.default_rng(0)
    every = np.arange(65536, dtype=np.uint16)                     # every bf16 pattern, in runs of 8
    shuffled = rng.permutation(every)
    scales = np.exp2(rng.integers(-30, 30, 4096 * 8)).astype(np.float32)
    mixed = oracle.bf16_bits(rng.standard_normal(4096 * 8).astype(np.float32) * scales)
    for name, arr in (("every pattern", every), ("shuffled", shuffled), ("mixed scales", mixed)):
        src = dev(arr)
        dst = dev_zeros(arr.shape)
        assert hip.xdna_bfp16_quantize8_bf16(ptr(src), ptr(dst), arr.size // 8, stream()) == 0
        np.testing.assert_array_equal(host(dst), oracle.bfp16_quantize8(arr), err_msg=name)
        # in place
        assert hip.xdna_bfp16_quantize8_bf16(ptr(src), ptr(src), arr.size // 8, stream()) == 0
        np.testing.assert_array_equal(host(src), host(dst), err_msg=name + " in place")
    misaligned = dev_zeros((24,))
    assert hip.xdna_bfp16_quantize8_bf16(ptr(misaligned) + 2, ptr(misaligned), 1, stream()) == -1


@pytest.mark.parametrize("cin,cout", [(64, 128), (130, 40), (3, 64), (200, 300)])
def test_quantized_prepared_weights_are_the_codec_decoded(hip, cin, cout):
    """The prepared weight forms, quantized, equal what the GPU codec kernels encode and
    decode (forward and dX forms, every 128-channel block)."""
    rng = np.random.default_rng(cin + cout)
    w = oracle.bf16_bits((rng.standard_normal((cout, cin, 3, 3)) * np.exp2(rng.integers(-6, 3, (cout, cin, 1, 1))))
                         .astype(np.float32))
    wd = dev(w)
    for dx, (ci, co) in ((0, (cin, cout)), (1, (cout, cin))):
        nbytes = hip.xdna_conv3x3_prepared_weight_bytes(ci, co)
        wt = dev_zeros((nbytes // 2,))
        assert hip.xdna_conv3x3_prepare_weights_bf16(ptr(wd), ptr(wt), cout, cin, dx, stream()) == 0
        assert hip.xdna_bfp16_quantize8_bf16(ptr(wt), ptr(wt), nbytes // 16, stream()) == 0
        chunks = -(-ci // 64)
        q = host(wt).reshape(-1, chunks * 9, 64)
        blk = hip.xdna_conv3x3w_weights_bfp16_bytes(chunks)
        enc = dev_zeros(((blk + 1) // 2,))
        dec = torch.zeros(blk // 9 * 8, dtype=torch.float32, device="cuda")
        for nb in range(-(-co // 128)):
            if dx:
                assert hip.xdna_conv3x3w_pack_weights_dx_bfp16(ptr(wd), ptr(enc), cout, cin, chunks, nb, stream()) == 0
            else:
                assert hip.xdna_conv3x3w_pack_weights_bfp16(ptr(wd), ptr(enc), cout, cin, chunks, nb, stream()) == 0
            assert hip.xdna_bfp16_decode_f32(ptr(enc), ptr(dec), blk // 9, stream()) == 0
            d = host(dec).reshape(chunks * 9, 8, 8, 2, 8, 8).transpose(1, 3, 4, 0, 2, 5).reshape(128, chunks * 9, 64)
            want = (d.view(np.uint32) >> 16).astype(np.uint16)
            rows = min(128, co - 128 * nb)
            np.testing.assert_array_equal(q[128 * nb:128 * nb + rows], want[:rows], err_msg=f"dx {dx} block {nb}")


def _data(B, Cin, Cout, H, W, seed):
    rng = np.random.default_rng(seed)
    bound = np.sqrt(6.0 / (9 * Cin))
    x = oracle.rng_bf16(rng, (B, Cin, H, W))
    w = oracle.bf16_bits(rng.uniform(-bound, bound, (Cout, Cin, 3, 3)).astype(np.float32))
    b = oracle.bf16_bits(rng.uniform(-0.1, 0.1, (Cout,)).astype(np.float32))
    dy = oracle.rng_bf16(rng, (B, Cout, H, W))
    return x, w, b, dy


def _emul(hip, src, w, bias, B, cin, cout, H, W, dgrad, act=0):
    """The C-ABI emulated conv of NCHW `src` (cin channels) with the forward weight `w`
    (dgrad: its flip + swap form), through the tight layout."""
    pb = hip.xdna_conv3x3_layout_packed_bytes(B, cin, H, W, TIGHT)
    packed = dev_zeros((pb // 2,))
    assert hip.xdna_conv3x3_layout_pack_bf16(ptr(dev(src)), ptr(packed), B, cin, H, W, TIGHT, stream()) == 0
    wb = hip.xdna_conv3x3_prepared_weight_bytes(cin, cout)
    wt = dev_zeros((wb // 2,))
    Co, Ci = (cin, cout) if dgrad else (cout, cin)  # the forward weight's [Cout][Cin]
    assert hip.xdna_conv3x3_prepare_weights_bf16(ptr(dev(w)), ptr(wt), Co, Ci, int(dgrad), stream()) == 0
    y = dev_zeros((B, cout, H, W))
    bd = dev(bias) if bias is not None else None
    assert hip.xdna_conv3x3_layout_rows_bfp16_emul_bf16(ptr(packed), ptr(wt), ptr(bd), ptr(y), B, cin, cout, H, W,
                                                        TIGHT, act, stream()) == 0
    return host(y)


SHAPES = [
    (2, 64, 64, 12, 12),
    (3, 70, 130, 9, 11),
    (2, 3, 32, 7, 5),
    (1, 64, 64, 8, 40),     # two width strips
    (2, 128, 96, 36, 36),
    (1, 256, 64, 18, 18),
    (4, 32, 48, 9, 9),
    (6, 64, 80, 36, 36),    # several 2048-row groups
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_emulated_conv_matches_oracle(hip, shape):
    B, Cin, Cout, H, W = shape
    print(f"bfp16 emulation {shape}", flush=True)
    x, w, b, dy = _data(*shape, seed=sum(shape) + 7)
    y = _emul(hip, x, w, b, B, Cin, Cout, H, W, dgrad=False)
    _agree(y, oracle.conv3x3_bfp16_emul(x, w, b), f"fwd {shape}")
    gx = _emul(hip, dy, w, None, B, Cout, Cin, H, W, dgrad=True)
    _agree(gx, oracle.conv3x3_dgrad_bfp16_emul(dy, w), f"dgrad {shape}")


def test_emulated_conv_relu_epilogue(hip):
    B, Cin, Cout, H, W = 2, 64, 64, 18, 18
    x, w, b, _ = _data(B, Cin, Cout, H, W, seed=11)
    y = _emul(hip, x, w, b, B, Cin, Cout, H, W, dgrad=False)
    yr = _emul(hip, x, w, b, B, Cin, Cout, H, W, dgrad=False, act=1)
    v = oracle.bf16_value(y)
    want = np.where(np.isnan(v) | (v > 0), y, np.uint16(0))
    np.testing.assert_array_equal(yr, want)


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.fixture
def emulation():
    xdna_train.set_npu_mode(2)
    xdna_train.set_bfp16_emulation(True)
    try:
        yield
    finally:
        xdna_train.set_bfp16_emulation(False)


def test_aten_route(emulation):
    """With the mode on, nn.Conv2d's forward and input gradient run the emulation and its
    weight and bias gradients stay exact; a stride-2 conv is not emulated (the reference's
    NPU takes only stride-1 convs); with the mode off nothing is emulated."""
    assert xdna_train.bfp16_emulation()
    torch.manual_seed(5)
    conv = nn.Conv2d(64, 40, 3, padding=1).bfloat16()
    x = torch.randn(3, 64, 20, 20).bfloat16()
    dy = torch.randn(3, 40, 20, 20).bfloat16()
    cd = nn.Conv2d(64, 40, 3, padding=1).bfloat16().to(X)
    cd.load_state_dict(conv.state_dict())
    xdna_train.reset_mapped_cpu_stats()
    xd = x.to(X).requires_grad_()
    yd = cd(xd)
    yd.backward(dy.to(X))
    torch.xdna.synchronize()
    st = xdna_train.mapped_cpu_stats()
    assert st.get("hip_conv3x3.bfp16_emul.fwd.run", {}).get("calls", 0) == 1, st
    assert st.get("hip_conv3x3.bfp16_emul.dx.run", {}).get("calls", 0) == 1, st
    xb, wb, bb, dyb = (_bits(t) for t in (x, conv.weight, conv.bias, dy))
    _agree(_bits(yd), oracle.conv3x3_bfp16_emul(xb, wb, bb), "aten fwd")
    _agree(_bits(xd.grad), oracle.conv3x3_dgrad_bfp16_emul(dyb, wb), "aten dgrad")
    gw, gb = oracle.conv3x3_wgrad(xb, dyb)
    check_bf16(_bits(cd.weight.grad), gw, what="aten wgrad (exact)")
    check_bf16(_bits(cd.bias.grad), gb, what="aten bias grad (exact)")

    s2 = nn.Conv2d(32, 16, 3, stride=2, padding=1).bfloat16().to(X)
    xdna_train.reset_mapped_cpu_stats()
    y2 = s2(torch.randn(2, 32, 12, 12).bfloat16().to(X).requires_grad_())
    y2.sum().backward()
    torch.xdna.synchronize()
    st = xdna_train.mapped_cpu_stats()
    assert st.get("hip_conv3x3_s2.fwd.run", {}).get("calls", 0) == 1, st
    assert not any("bfp16_emul" in k for k in st), st

    xdna_train.set_bfp16_emulation(False)
    xdna_train.reset_mapped_cpu_stats()
    cd(xd).sum().backward()
    torch.xdna.synchronize()
    assert not any("bfp16_emul" in k for k in xdna_train.mapped_cpu_stats())


def test_style_training_with_emulation_follows_bf16(emulation):
    """The reference's precision gate (benchmarks/bfp16_training_gate.py:120-160) on BASELINE
    config 4's network: 60 steps with the emulation and without (both on xdna), with the
    gate's optimizer (Adam, lr 1e-4, weight decay 1e-5); windowed means of the loss within
    2 % (the reference's 300-step gate: windows within +-0.5 %, one at 1.4 %,
    benchmarks/results/bfp16_gate.log).  At config 4's own lr of 1e-3 the run is too
    sensitive to rounding for such a comparison (the CPU's runs one bf16 ulp apart already
    differ by ~3 %, tests/test_gpu_loss_curves.py).  The emulated step runs every eligible
    conv through the emulation."""
    import bench
    import statistics

    def curve(on):
        xdna_train.set_bfp16_emulation(on)
        step, _ = bench.build_style(torch, X, fused=None, lr=1e-4, weight_decay=1e-5)
        return [float(step().detach()) for _ in range(60)]

    xdna_train.reset_mapped_cpu_stats()
    emu = curve(True)
    st = xdna_train.mapped_cpu_stats()
    assert st.get("hip_conv3x3.bfp16_emul.fwd.run", {}).get("calls", 0) >= 60 * 10, st
    base = curve(False)
    wins = [(statistics.mean(base[i:i + 10]), statistics.mean(emu[i:i + 10])) for i in range(0, 60, 10)]
    gaps = [abs(e - b) / b for b, e in wins]
    print("bf16 / emulated windows:", [(f"{b:.5g}", f"{e:.5g}") for b, e in wins], flush=True)
    print("gaps:", [f"{g:.2%}" for g in gaps], flush=True)
    assert emu[-1] < emu[0]
    assert max(gaps) <= 0.02, gaps
