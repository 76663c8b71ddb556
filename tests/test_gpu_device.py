"""The xdna PrivateUse1 device on an MI355X: a torch.device("xdna") script runs
unchanged, the hot ops run the HIP kernels (proved by the path counters, as the
reference's tests do with npu_conv3x3w.*.run: run_conv3x3w_torch.py:181-186), and the
results match PyTorch's CPU bf16 path (the reference's numerical target).

Ported semantics: deferred-dW snapshot (run_deferred_dw.py:62-71), GEMM storage
offsets and recycled buffers (run_gemm_safety.py:44-87), exact out= variants
(test_device_physical.py:118-178), fused Adam parity (training_interfaces.py:25-37),
the 40-step CPU-vs-device training check (quick_check.py:34-84).
"""
import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

import oracle
import xdna_train  # noqa: F401  (registers the xdna device)
from gpu_util import check_bf16

pytestmark = pytest.mark.gpu

X = torch.device("xdna")


@pytest.fixture(scope="module", autouse=True)
def xdna():
    import xdna_train

    assert xdna_train.is_available(), "xdna device not available on the GPU box"
    xdna_train.set_npu_mode(2)
    return xdna_train


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def test_tensor_basics(xdna):
    a = torch.arange(12, dtype=torch.float32).reshape(3, 4)
    d = a.to(X)
    assert d.device.type == "xdna"
    assert torch.equal(d.cpu(), a)
    assert torch.equal((d * 2 + 1).cpu(), a * 2 + 1)
    assert torch.equal(d.t().contiguous().cpu(), a.t().contiguous())
    assert torch.equal(d[1:, ::2].cpu(), a[1:, ::2])
    d.add_(1)
    assert torch.equal(d.cpu(), a + 1)
    assert float(d.sum().item()) == float((a + 1).sum())
    z = torch.zeros(5, 6, device=X, dtype=torch.bfloat16)
    assert z.device.type == "xdna" and not z.cpu().any()
    r = torch.randn(100, device=X)
    assert r.device.type == "xdna" and r.cpu().std() > 0.5
    c = torch.cat([d, d], 0)
    assert torch.equal(c.cpu(), torch.cat([a + 1, a + 1], 0))
    out = torch.empty(0, device=X)
    torch.add(d, d, out=out)  # out= resize through the fallback
    assert out.shape == (3, 4) and torch.equal(out.cpu(), 2 * (a + 1))
    assert "xdna" in repr(d) or "device='xdna:0'" in repr(d)


def test_conv_forward_backward_matches_cpu_and_oracle(xdna):
    xdna.reset_mapped_cpu_stats()
    torch.manual_seed(0)
    conv = nn.Conv2d(64, 96, 3, padding=1).bfloat16()
    x = torch.randn(4, 64, 20, 24).bfloat16()
    dy = torch.randn(4, 96, 20, 24).bfloat16()
    cd = nn.Conv2d(64, 96, 3, padding=1).bfloat16().to(X)
    cd.load_state_dict(conv.state_dict())
    xd = x.to(X).requires_grad_()
    yd = cd(xd)
    yd.backward(dy.to(X))
    st = xdna.mapped_cpu_stats()
    for k in ("hip_conv3x3.fwd.run", "hip_conv3x3.dx.run", "hip_conv3x3.dw.run"):
        assert st.get(k, {}).get("calls", 0) >= 1, (k, st)
    xb, wb, bb, dyb = (bits(t) for t in (x, conv.weight, conv.bias, dy))
    check_bf16(bits(yd), oracle.conv3x3_fwd(xb, wb, bb), what="fwd")
    check_bf16(bits(xd.grad), oracle.conv3x3_dgrad(dyb, wb), what="dgrad")
    gw, gb = oracle.conv3x3_wgrad(xb, dyb)
    check_bf16(bits(cd.weight.grad), gw, what="wgrad")
    check_bf16(bits(cd.bias.grad), gb, what="bias grad")
    # against the CPU bf16 path (the reference's target): rel L2 <= 1e-2
    xc = x.clone().requires_grad_()
    yc = conv(xc)
    yc.backward(dy)
    for got, ref in ((yd, yc), (xd.grad, xc.grad), (cd.weight.grad, conv.weight.grad)):
        g, r = got.detach().cpu().float(), ref.detach().float()
        assert (g - r).norm() / r.norm() < 1e-2


@pytest.mark.parametrize("shape", [(4, 64, 96, 20, 24), (2, 32, 48, 12, 72), (1, 160, 144, 5, 72),
                                   (1, 16, 24, 6, 150), (1, 8, 16, 3, 300)],
                         ids=lambda s: "x".join(map(str, s)))
def test_wgrad_forms(xdna, shape):
    """Both 3x3 weight-gradient forms (channel-major copies; packed rows sharing the input
    gradient's packed dY) through the op path against the oracle; images wider than 142
    take the rows form whatever the setting."""
    B, Cin, Cout, H, W = shape
    print(f"wgrad forms {shape}", flush=True)
    g = torch.Generator().manual_seed(sum(shape))
    x = torch.randn(B, Cin, H, W, generator=g).bfloat16()
    dy = torch.randn(B, Cout, H, W, generator=g).bfloat16()
    w = (torch.randn(Cout, Cin, 3, 3, generator=g) * 0.05).bfloat16()
    gw_ref, gb_ref = oracle.conv3x3_wgrad(bits(x), bits(dy))
    gx_ref = oracle.conv3x3_dgrad(bits(dy), bits(w))
    expect_rows = {1: W > 142, 2: True, 0: True}
    try:
        for form in (1, 2, 0):
            xdna.set_wgrad_form(form)
            assert xdna.wgrad_form() == form
            xdna.reset_mapped_cpu_stats()
            wd = w.to(X).requires_grad_()
            bd = torch.zeros(Cout, dtype=torch.bfloat16).to(X).requires_grad_()
            xd = x.to(X).requires_grad_()
            torch.nn.functional.conv2d(xd, wd, bd, padding=1).backward(dy.to(X))
            st = xdna.mapped_cpu_stats()
            assert st.get("hip_conv3x3.dw.run", {}).get("calls", 0) == 1, st
            assert st.get("hip_conv3x3.dw_rows.run", {}).get("calls", 0) == int(expect_rows[form]), (form, st)
            # the rows form reads the forward's packed input
            assert st.get("hip_conv3x3.dw_rows.kept_pack", {}).get("calls", 0) == int(expect_rows[form]), st
            check_bf16(bits(wd.grad), gw_ref, what=f"wgrad form {form}")
            check_bf16(bits(bd.grad), gb_ref, what=f"bias grad form {form}")
            check_bf16(bits(xd.grad), gx_ref, what=f"dgrad form {form}")
    finally:
        xdna.set_wgrad_form(0)


def test_kept_packed_input_shared_and_stale(xdna):
    """Two convs reading one input (one kept pack, taken by the first backward; the second
    packs again), and a forward whose backward never runs: gradients still match the
    oracle."""
    g = torch.Generator().manual_seed(21)
    x = torch.randn(2, 32, 10, 12, generator=g).bfloat16()
    w1 = (torch.randn(48, 32, 3, 3, generator=g) * 0.05).bfloat16()
    w2 = (torch.randn(40, 32, 3, 3, generator=g) * 0.05).bfloat16()
    d1 = torch.randn(2, 48, 10, 12, generator=g).bfloat16()
    d2 = torch.randn(2, 40, 10, 12, generator=g).bfloat16()
    xd = x.to(X)
    w1d, w2d = w1.to(X).requires_grad_(), w2.to(X).requires_grad_()
    # a forward without a backward leaves an entry behind
    F.conv2d(xd, w1d, padding=1)
    xdna.reset_mapped_cpu_stats()
    y1 = F.conv2d(xd, w1d, padding=1)
    y2 = F.conv2d(xd, w2d, padding=1)
    torch.autograd.backward([y1, y2], [d1.to(X), d2.to(X)])
    st = xdna.mapped_cpu_stats()
    assert st.get("hip_conv3x3.dw_rows.run", {}).get("calls", 0) == 2, st
    assert st.get("hip_conv3x3.dw_rows.kept_pack", {}).get("calls", 0) == 1, st
    for wd, d in ((w1d, d1), (w2d, d2)):
        gw_ref, _ = oracle.conv3x3_wgrad(bits(x), bits(d))
        check_bf16(bits(wd.grad), gw_ref, what="wgrad shared input")
    xdna.empty_cache()


@pytest.mark.parametrize("offset", [0, 1, 4], ids=lambda o: f"bias_offset{o}")
@pytest.mark.parametrize("cout", [64, 66])
def test_conv_bias_views(xdna, offset, cout):
    """Conv bias as a view into a larger tensor: 8-byte aligned (offset 0, 4: 4-channel
    vector loads when cout % 4 == 0) and 2-byte aligned (offset 1: per-row loads), against
    the oracle, on the main and the small-grid kernels."""
    g = torch.Generator().manual_seed(31 + offset + cout)
    for (B, H, W) in ((2, 12, 12), (16, 36, 36)):
        x = torch.randn(B, 48, H, W, generator=g).bfloat16()
        w = (torch.randn(cout, 48, 3, 3, generator=g) * 0.05).bfloat16()
        big = torch.randn(cout + 8, generator=g).bfloat16()
        bias = big[offset:offset + cout]
        ref = oracle.conv3x3_fwd(bits(x), bits(w), bits(bias))
        bd = big.to(X)[offset:offset + cout]
        assert bd.data_ptr() % 8 == (2 * offset) % 8
        y = F.conv2d(x.to(X), w.to(X), bd, padding=1)
        check_bf16(bits(y), ref, what=f"conv with bias view (offset {offset}, cout {cout}, B {B})")


def test_other_convs_run_on_general_kernels(xdna):
    """5x5, 9x9 and 7x7-stride-2 convolutions (forward and backward) run on the general HIP
    kernels (mode 2: always), 1x1 ones on the 1x1 GEMM path, the 3x3 / stride-2 / pad-1 one
    on the stride-1 3x3 path, and all match the CPU bf16 path and the float64 oracle."""
    xdna.reset_mapped_cpu_stats()
    xdna.set_general_conv_mode(2)
    specs = [(8, 16, 5, 1, 2), (8, 16, 3, 2, 1), (8, 16, 1, 1, 0), (3, 32, 9, 1, 4), (3, 16, 7, 2, 3),
             (16, 24, 1, 2, 0)]
    for cin, cout, k, s, pd in specs:
        torch.manual_seed(k * 10 + s)
        conv = nn.Conv2d(cin, cout, k, stride=s, padding=pd).bfloat16()
        x = torch.randn(2, cin, 14, 13).bfloat16()
        cd = nn.Conv2d(cin, cout, k, stride=s, padding=pd).bfloat16().to(X)
        cd.load_state_dict(conv.state_dict())
        xd = x.to(X).requires_grad_()
        yd = cd(xd)
        dy = torch.randn(yd.shape).bfloat16()
        yd.backward(dy.to(X))
        xb, wb, bb, dyb = (bits(t) for t in (x, conv.weight, conv.bias, dy))
        what = f"k{k} s{s} {cin}->{cout}"
        check_bf16(bits(yd), oracle.conv2d_fwd(xb, wb, bb, (s, s), (pd, pd)), what=f"fwd {what}")
        check_bf16(bits(xd.grad), oracle.conv2d_dgrad(dyb, wb, (14, 13), (s, s), (pd, pd)), what=f"dgrad {what}")
        gw, gb = oracle.conv2d_wgrad(xb, dyb, (k, k), (s, s), (pd, pd))
        check_bf16(bits(cd.weight.grad), gw, what=f"wgrad {what}")
        check_bf16(bits(cd.bias.grad), gb, what=f"bias grad {what}")
        xc = x.clone().requires_grad_()
        yc = conv(xc)
        yc.backward(dy)
        for got, ref in ((yd, yc), (xd.grad, xc.grad), (cd.weight.grad, conv.weight.grad)):
            g, r = got.detach().cpu().float(), ref.detach().float()
            assert (g - r).norm() / r.norm() < 1e-2, what
    st = xdna.mapped_cpu_stats()
    for key in ("hip_conv2d.fwd.run", "hip_conv2d.dx.run", "hip_conv2d.dw.run"):
        assert st.get(key, {}).get("calls", 0) == 3, (key, st)  # 5x5, 9x9, 7x7 / stride 2
    for key in ("hip_conv1x1.fwd.run", "hip_conv1x1.bwd.run"):
        assert st.get(key, {}).get("calls", 0) == 2, (key, st)
    for key in ("hip_conv3x3_s2.fwd.run", "hip_conv3x3_s2.bwd.run"):
        assert st.get(key, {}).get("calls", 0) == 1, (key, st)
    assert "aten::convolution.rocm" not in st and "aten::convolution_backward.rocm" not in st


def _routed_conv(cin, cout, k, s, pd, B=2, H=12, W=10, seed=0):
    """One conv forward + backward on xdna from CPU-made bf16 operands; returns the path
    counters and the results checked against the float64 oracle."""
    torch.manual_seed(seed + cin + cout + k)
    conv = nn.Conv2d(cin, cout, k, stride=s, padding=pd).bfloat16()
    x = torch.randn(B, cin, H, W).bfloat16()
    cd = nn.Conv2d(cin, cout, k, stride=s, padding=pd).bfloat16().to(X)
    cd.load_state_dict(conv.state_dict())
    xdna_train.reset_mapped_cpu_stats()
    xd = x.to(X).requires_grad_()
    yd = cd(xd)
    dy = torch.randn(yd.shape).bfloat16()
    yd.backward(dy.to(X))
    torch.xdna.synchronize()
    st = xdna_train.mapped_cpu_stats()
    xb, wb, bb, dyb = (bits(t) for t in (x, conv.weight, conv.bias, dy))
    what = f"k{k} s{s} {cin}->{cout} B{B} {H}x{W}"
    check_bf16(bits(yd), oracle.conv2d_fwd(xb, wb, bb, (s, s), (pd, pd)), what=f"fwd {what}")
    check_bf16(bits(xd.grad), oracle.conv2d_dgrad(dyb, wb, (H, W), (s, s), (pd, pd)), what=f"dgrad {what}")
    gw, gb = oracle.conv2d_wgrad(xb, dyb, (k, k), (s, s), (pd, pd))
    check_bf16(bits(cd.weight.grad), gw, what=f"wgrad {what}")
    return st, bits(cd.bias.grad), gb, what


def test_default_routing_of_general_convs(xdna):
    """Mode 2 (default) runs every eligible conv direction on the HIP kernels, the style
    network's 9x9 32->3 gradients included (the few-output weight-gradient kernel and the
    gather input gradient); 3x3 / stride-2 layers take the stride-1 3x3 path; 3x3 layers
    with at most 4 input channels take the general forward and weight gradient and the
    3x3 input gradient, with 8 inputs the 3x3 path throughout.  Mode 1 keeps the gradients
    of few-output layers on MIOpen.  Every result matches the float64 oracle."""
    assert xdna.general_conv_mode() == 2
    hip_all = {"hip_conv2d.fwd.run": 1, "hip_conv2d.dw.run": 1, "hip_conv2d.dx.run": 1,
               "aten::convolution.rocm": 0, "aten::convolution_backward.rocm": 0}
    specs = [  # cin, cout, k, s, p, mode, expected counters
        (32, 3, 9, 1, 4, 2, hip_all),
        (3, 32, 9, 1, 4, 2, hip_all),
        (32, 64, 3, 2, 1, 2, {"hip_conv3x3_s2.fwd.run": 1, "hip_conv3x3_s2.bwd.run": 1,
                              "aten::convolution.rocm": 0, "aten::convolution_backward.rocm": 0}),
        (3, 64, 3, 1, 1, 2, {"hip_conv2d.fwd.run": 1, "hip_conv3x3.dx.run": 1, "hip_conv2d.dw.run": 1,
                             "hip_conv3x3.fwd.run": 0, "hip_conv3x3.dw.run": 0, "aten::convolution.rocm": 0,
                             "aten::convolution_backward.rocm": 0}),
        (4, 32, 3, 1, 1, 1, {"hip_conv2d.fwd.run": 1, "hip_conv3x3.dx.run": 1, "hip_conv2d.dw.run": 1,
                             "aten::convolution_backward.rocm": 0}),
        (8, 64, 3, 1, 1, 2, {"hip_conv3x3.fwd.run": 1, "hip_conv3x3.dx.run": 1, "hip_conv3x3.dw.run": 1,
                             "hip_conv2d.fwd.run": 0, "hip_conv2d.dw.run": 0}),
        (32, 3, 9, 1, 4, 1, {"hip_conv2d.fwd.run": 1, "aten::convolution_backward.rocm": 1}),
    ]
    try:
        for cin, cout, k, s, pd, mode, expect in specs:
            xdna.set_general_conv_mode(mode)
            st, gbd, gb, what = _routed_conv(cin, cout, k, s, pd)
            for key, n in expect.items():
                assert st.get(key, {}).get("calls", 0) == n, (cin, cout, mode, key, st)
            if mode == 2:
                check_bf16(gbd, gb, what=f"bias grad {what}")
            else:  # bias gradients from MIOpen sum in another order: relative bar
                g = oracle.bf16_value(gbd)
                assert np.abs(g - gb).max() <= 2 * oracle.bf16_ulp(np.abs(gb).max()) + 1e-6, what
    finally:
        xdna.set_general_conv_mode(2)


@pytest.mark.parametrize("cin,cout,k,pd,B,H,W", [
    (32, 3, 9, 4, 40, 36, 36),   # the style network's last layer at its training size
    (32, 3, 9, 4, 1, 7, 5),      # output narrower than the kernel
    (16, 1, 5, 2, 3, 17, 33),
    (48, 2, 7, 0, 2, 20, 19),    # no padding
    (4, 4, 3, 0, 5, 9, 130),     # wide rows: one staged input row per pass
    (64, 4, 7, 3, 2, 11, 11),    # 3136 taps: 13 per thread
    (3, 3, 9, 4, 2, 16, 16),
    (640, 1, 3, 0, 2, 6, 6),     # 1920 row pairs: four passes of 512 threads
    (8, 2, 11, 5, 2, 15, 14),    # wider than 9 and even widths: the per-tap form
    (16, 3, 4, 2, 2, 10, 12),
])
def test_few_output_weight_gradient(xdna, cin, cout, k, pd, B, H, W):
    """Stride-1 convs with at most 4 output channels take the few-output weight-gradient
    kernels (fp32 FMA over staged rows, fixed-order partial reduce; a sliding register
    window for odd widths up to 9, one sum per tap otherwise): weight and bias gradients
    match the float64 oracle to the conv bar, across kernel sizes, paddings, row widths and
    tap counts."""
    st, gbd, gb, what = _routed_conv(cin, cout, k, 1, pd, B=B, H=H, W=W, seed=5)
    check_bf16(gbd, gb, what=f"bias grad {what}")
    for key in ("hip_conv2d.dw.run", "hip_conv2d.dx.run"):
        assert st.get(key, {}).get("calls", 0) == 1, (key, st)
    assert "aten::convolution_backward.rocm" not in st


def test_trainable_weight_forms_follow_the_version(xdna):
    """The forward of a trainable weight prepares the input gradient's weight form too and
    leaves it for the backward; an in-place update of the weight (a version bump) between
    the two makes the backward prepare it again, so dx always uses the current weight."""
    torch.manual_seed(3)
    x = torch.randn(2, 64, 10, 10).bfloat16()
    dy = torch.randn(2, 64, 10, 10).bfloat16()
    w = (torch.randn(64, 64, 3, 3) * 0.05).bfloat16()
    wd = w.to(X).requires_grad_()
    xd, dyd = x.to(X), dy.to(X)
    args = ([1, 1], [1, 1], [1, 1], False, [0, 0], 1)
    with torch.no_grad():
        torch.ops.aten.convolution(xd, wd, None, *args)
        for step in range(2):
            dx = torch.ops.aten.convolution_backward(dyd, xd, wd, None, *args, [True, False, False])[0]
            ref = oracle.conv2d_dgrad(bits(dy), bits(wd), (10, 10), (1, 1), (1, 1))
            check_bf16(bits(dx), ref, what=f"dgrad after update {step}")
            wd.mul_(-0.5)  # version bump, no new forward


def test_ineligible_convs_fall_back(xdna):
    """Dilated, grouped and fp32 convolutions stay on PyTorch-ROCm."""
    xdna.reset_mapped_cpu_stats()
    for conv, dt in ((nn.Conv2d(8, 16, 3, padding=2, dilation=2), torch.bfloat16),
                     (nn.Conv2d(8, 16, 3, padding=1, groups=2), torch.bfloat16),
                     (nn.Conv2d(8, 16, 3, padding=1), torch.float32)):
        conv = conv.to(dt)
        x = torch.randn(2, 8, 10, 10).to(dt)
        cd = nn.Conv2d(8, 16, 3, padding=conv.padding, dilation=conv.dilation, groups=conv.groups).to(dt).to(X)
        cd.load_state_dict(conv.state_dict())
        y = cd(x.to(X))
        ref = conv(x)
        assert (y.cpu().float() - ref.float()).norm() / ref.float().norm() < 1e-2
    st = xdna.mapped_cpu_stats()
    assert "hip_conv3x3.fwd.run" not in st and "hip_conv2d.fwd.run" not in st
    assert st["aten::convolution.rocm"]["calls"] == 3


def test_deferred_wgrad_snapshots_inputs(xdna):
    """Writing x or dY after backward must not change the weight gradient."""
    torch.manual_seed(1)
    conv = nn.Conv2d(32, 32, 3, padding=1).bfloat16().to(X)
    x = torch.randn(2, 32, 16, 16).bfloat16().to(X)
    dy = torch.randn(2, 32, 16, 16).bfloat16().to(X)
    y = conv(x)
    (gw1,) = torch.autograd.grad(y, conv.weight, dy, retain_graph=True)
    ref = bits(gw1).copy()
    y2 = conv(x)
    (gw2,) = torch.autograd.grad(y2, conv.weight, dy)
    x.mul_(3.0)
    dy.zero_()
    np.testing.assert_array_equal(bits(gw2), ref)


def test_linear_and_gemm_ops(xdna):
    xdna.reset_mapped_cpu_stats()
    torch.manual_seed(2)
    lin = nn.Linear(256, 192).bfloat16()
    ld = nn.Linear(256, 192).bfloat16().to(X)
    ld.load_state_dict(lin.state_dict())
    x = torch.randn(130, 256).bfloat16()
    dy = torch.randn(130, 192).bfloat16()
    xd = x.to(X).requires_grad_()
    yd = ld(xd)
    yd.backward(dy.to(X))
    st = xdna.mapped_cpu_stats()
    assert st.get("hip_gemm.addmm.run", {}).get("calls", 0) >= 1, st
    assert st.get("hip_gemm.mm.run", {}).get("calls", 0) >= 2, st
    xb, wb, bb, db = (bits(t) for t in (x, lin.weight, lin.bias, dy))
    check_bf16(bits(yd), oracle.gemm(xb, wb.T, bb), what="linear fwd")
    check_bf16(bits(xd.grad), oracle.gemm(db, wb), what="linear dX")
    check_bf16(bits(ld.weight.grad), oracle.gemm(db.T, xb), what="linear dW")
    # bmm (Gram matrices) and 3-D linear inputs
    f = torch.randn(5, 24, 49).bfloat16()
    g = torch.bmm(f.to(X), f.to(X).transpose(1, 2))
    check_bf16(bits(g), oracle.gemm(bits(f), np.swapaxes(bits(f), 1, 2)), what="bmm")
    y3 = ld(torch.randn(3, 7, 256).bfloat16().to(X))
    assert y3.shape == (3, 7, 192)


def test_gemm_storage_offsets_and_recycled_buffers(xdna):
    """Identity products are exact, also for operands that start inside an allocation
    and outputs written into recycled (dirty) memory (run_gemm_safety.py:44-83)."""
    eye = torch.eye(64, dtype=torch.bfloat16)
    base = torch.randn(65, 64).bfloat16()
    for _ in range(3):
        junk = torch.full((64, 64), float("nan"), dtype=torch.bfloat16, device=X)
        del junk
        a = base.to(X)[1:]
        out = a @ eye.to(X)
        assert torch.equal(out.cpu(), base[1:])
        out2 = eye.to(X) @ a
        assert torch.equal(out2.cpu(), base[1:])
    # exact out= variants
    a = torch.randn(8, 16).bfloat16()
    b = torch.randn(16, 4).bfloat16()
    o = torch.empty(2, 2, dtype=torch.bfloat16, device=X)
    torch.mm(a.to(X), b.to(X), out=o)
    assert o.shape == (8, 4)
    assert torch.equal(o.cpu(), torch.mm(a.to(X), b.to(X)).cpu())


def test_fused_adam_bitwise_vs_cpu(xdna):
    torch.manual_seed(3)
    ps = [torch.randn(300, 7).bfloat16(), torch.randn(1000).bfloat16()]
    pc = [nn.Parameter(p.clone()) for p in ps]
    pd = [nn.Parameter(p.clone().to(X)) for p in ps]
    oc = torch.optim.Adam(pc, lr=1e-3, fused=True)
    od = torch.optim.Adam(pd, lr=1e-3)  # fused by the xdna pre-hook
    xdna.reset_mapped_cpu_stats()
    for step in range(3):
        grads = [torch.randn_like(p) * 0.01 for p in ps]
        for p, g in zip(pc, grads):
            p.grad = g.clone()
        for p, g in zip(pd, grads):
            p.grad = g.clone().to(X)
        oc.step()
        od.step()
    assert od.param_groups[0]["fused"] is True
    assert xdna.mapped_cpu_stats()["hip_adam.run"]["calls"] == 3
    for a, b in zip(pc, pd):
        np.testing.assert_array_equal(bits(a), bits(b))


def test_param_identity_across_to(xdna):
    m = nn.Linear(4, 4).bfloat16()
    opt = torch.optim.Adam(m.parameters())
    w = m.weight
    m.to(X)
    assert m.weight is w and w.device.type == "xdna"
    m(torch.randn(2, 4).bfloat16().to(X)).sum().backward()
    before = w.detach().cpu().clone()
    opt.step()
    assert not torch.equal(w.detach().cpu(), before)


def test_c1_training_matches_cpu(xdna):
    """BASELINE config 1 (Conv2d 128->128 on [16,128,36,36], MSE to zeros, Adam 1e-3),
    5 steps on xdna and on CPU bf16 from the same seed: losses agree within 1 %."""
    def run(device):
        torch.manual_seed(0)
        model = nn.Conv2d(128, 128, 3, padding=1).bfloat16().to(device)
        x = torch.randn(16, 128, 36, 36).bfloat16().to(device)
        target = torch.zeros(16, 128, 36, 36, dtype=torch.bfloat16).to(device)
        opt = torch.optim.Adam(model.parameters(), lr=1e-3, betas=(0.9, 0.999), eps=1e-8,
                               fused=True)
        losses = []
        for _ in range(5):
            opt.zero_grad()
            loss = F.mse_loss(model(x).float(), target.float())
            loss.backward()
            opt.step()
            losses.append(float(loss.item()))
        return losses

    lc = run(torch.device("cpu"))
    ld = run(X)
    for a, b in zip(lc, ld):
        assert abs(a - b) <= 0.01 * abs(a), (lc, ld)
    assert ld[-1] < ld[0]


def test_launch_errors_raise(xdna):
    from xdna_train import device as dev

    conv = nn.Conv2d(16, 16, 3, padding=1).bfloat16().to(X)
    x = torch.randn(1, 16, 8, 8).bfloat16().to(X)
    dev.native().inject_failure(1, False)
    try:
        with pytest.raises(RuntimeError, match="injected failure"):
            conv(x)
    finally:
        dev.native().reset_failure_state()
    assert conv(x).shape == (1, 16, 8, 8)


def test_foreach_add_steps_one_launch():
    ts = [torch.zeros((), device=X) for _ in range(70)] + [torch.arange(5.0).to(X)]
    xdna_train.reset_mapped_cpu_stats()
    torch._foreach_add_(ts, 1)
    torch._foreach_add_(ts, 0.5)
    stats = xdna_train.mapped_cpu_stats()
    assert stats.get("hip_foreach_add.run", {}).get("calls", 0) == 2, stats
    assert all(float(t) == 1.5 for t in ts[:70])
    assert torch.equal(ts[70].cpu(), torch.arange(5.0) + 1.5)
    # bf16 lists take the ROCm path
    b = [torch.ones(3, device=X).bfloat16()]
    torch._foreach_add_(b, 2)
    assert torch.equal(b[0].cpu().float(), torch.full((3,), 3.0))


def test_frozen_weights_prepared_once_and_refreshed_on_write():
    torch.manual_seed(3)
    conv = torch.nn.Conv2d(64, 64, 3, padding=1).bfloat16()
    for p in conv.parameters():
        p.requires_grad_(False)
    x = torch.randn(2, 64, 10, 10).bfloat16()
    cd = torch.nn.Conv2d(64, 64, 3, padding=1).bfloat16()
    cd.load_state_dict(conv.state_dict())
    for p in cd.parameters():
        p.requires_grad_(False)
    cd = cd.to(X)
    xd = x.to(X)
    y1 = cd(xd)
    n0 = xdna_train.device.native().launch_count()
    y2 = cd(xd)
    n1 = xdna_train.device.native().launch_count()
    assert torch.equal(y1.cpu(), y2.cpu())
    # the second call reuses the prepared weights: the conv only (no preparation launch; a
    # frozen conv on a grid this small reads its NCHW input in place, with no pack launch)
    assert n1 - n0 == 1, (n0, n1)
    ref = conv(x).float()
    assert torch.allclose(y2.cpu().float(), ref, atol=5e-2, rtol=5e-2)
    # an in-place write bumps the version: the new weights are used
    with torch.no_grad():
        cd.weight.mul_(-1)
        conv.weight.mul_(-1)
    y3 = cd(xd)
    assert torch.allclose(y3.cpu().float(), conv(x).float(), atol=5e-2, rtol=5e-2)
    assert not torch.allclose(y3.cpu().float(), y2.cpu().float(), atol=5e-2, rtol=5e-2)


def test_non_default_stream_is_refused(xdna):
    """The device's caching allocator orders every use of a block on one stream, so xdna
    work on a side stream raises (instead of racing a recycled block); the default stream
    keeps working afterwards, and a graph capture (on its own capturing stream) is allowed."""
    a = torch.ones(1024, device=X)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        with pytest.raises(RuntimeError, match="default one is not supported"):
            (a + 1).cpu()
    torch.cuda.synchronize()
    assert float((a + 1).sum().cpu()) == 2048.0
    g = xdna.Graph()
    b = torch.zeros(1024, device=X)
    with xdna.graph(g):
        b.add_(a)
    g.replay()
    g.replay()
    torch.xdna.synchronize()
    assert float(b.sum().cpu()) == 2048.0


def test_mse_loss_without_resized_outputs():
    """mse_loss runs PyTorch-ROCm's functional kernel (not the out= form through the
    composite, which resized a 0-dim output), for every reduction, forward and backward."""
    import warnings
    g = torch.Generator().manual_seed(11)
    a = torch.randn(4, 8, 6, 6, generator=g)
    b = torch.randn(4, 8, 6, 6, generator=g)
    for red in ("mean", "sum", "none"):
        ad = a.to(X).requires_grad_()
        with warnings.catch_warnings(record=True) as w:
            warnings.simplefilter("always")
            out = torch.nn.functional.mse_loss(ad, b.to(X), reduction=red)
            out.sum().backward() if red == "none" else out.backward()
        assert not [x for x in w if "resized" in str(x.message)], [str(x.message) for x in w]
        ac = a.clone().requires_grad_()
        ref = torch.nn.functional.mse_loss(ac, b, reduction=red)
        ref.sum().backward() if red == "none" else ref.backward()
        assert out.shape == ref.shape and out.device.type == "xdna"
        torch.testing.assert_close(out.detach().cpu(), ref.detach(), rtol=1e-5, atol=1e-6)
        torch.testing.assert_close(ad.grad.cpu(), ac.grad, rtol=1e-5, atol=1e-6)
