"""The fused frozen-feature region on the GPU (the reference's regions.py:1-425 contract:
bf16 storage, fp32 arithmetic, one rounding; PyTorch's max-pool and ReLU-mask rules).

* Conv + ReLU in one epilogue equals the unfused xdna conv followed by relu, bit for bit.
* The region's max-pool equals torch.max_pool2d (PyTorch-ROCm on the same data), ties,
  NaN (as NaN: the encodings differ), -inf and odd sizes included; its backward pass routes each pooled gradient to the
  same element as PyTorch's max_pool2d backward and masks as threshold_backward does, bit
  for bit.
* Loss partials and the finishing sum against float64 sums; the Gram gradient against its
  formula in float64.
* End to end on a small VGG chain and at the BASELINE style configuration's shapes: the
  region's loss and dX against the eager ops in fp32 on the CPU (same bf16 inputs and
  weights), with path counters proving the region kernels ran; the reference's
  fuse_perceptual_loss pattern; and a captured step replayed.
"""
import numpy as np
import pytest
import torch
import torch.nn as nn

import bench
import xdna_train
from xdna_train import regions

pytestmark = pytest.mark.gpu
X = torch.device("xdna")


@pytest.fixture(scope="module", autouse=True)
def xdna():
    assert xdna_train.is_available(), "xdna device not available on the GPU box"
    xdna_train.set_npu_mode(2)
    return xdna_train


def C():
    return xdna_train.device.native()


def rocm(t):
    return C().cuda_alias(t)


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy()


def test_conv_relu_epilogue_is_relu_of_conv_bit_exact():
    g = torch.Generator().manual_seed(3)
    for (B, cin, cout, H, W) in ((2, 16, 32, 9, 9), (4, 64, 64, 18, 18), (2, 32, 48, 36, 37), (1, 8, 8, 72, 72)):
        x = torch.randn(B, cin, H, W, generator=g).bfloat16().to(X)
        w = (torch.randn(cout, cin, 3, 3, generator=g) * 0.1).bfloat16().to(X)
        b = torch.randn(cout, generator=g).bfloat16().to(X)
        y = C().region_conv3x3(x, w, b, 1)
        ref = torch.relu(C().region_conv3x3(x, w, b, 0))
        np.testing.assert_array_equal(bits(y), bits(ref), err_msg=str((B, cin, cout, H, W)))
        assert (bits(y) != np.int16(-32768)).all()  # relu(-0) is +0


def _special(shape, g):
    v = torch.randn(shape, generator=g)
    v = torch.round(v * 4) / 4  # many ties inside windows
    flat = v.view(-1)
    flat[::97] = float("-inf")
    flat[5::211] = float("nan")
    flat[7::53] = -0.0
    return v.bfloat16()


@pytest.mark.parametrize("shape", [(2, 3, 8, 8), (1, 5, 7, 9), (3, 16, 36, 36), (2, 4, 3, 6)])
def test_maxpool2_matches_torch(shape):
    g = torch.Generator().manual_seed(sum(shape))
    x = _special(shape, g).to(X)
    y = C().region_maxpool2(x)
    ref = torch.nn.functional.max_pool2d(rocm(x), 2, 2)
    # NaN where PyTorch has NaN (the encodings differ: PyTorch-ROCm writes 0xFFFF, this
    # kernel the canonical 0x7FC0), every other element bit for bit
    yn, rn = torch.isnan(y.cpu().float()), torch.isnan(ref.cpu().float())
    assert torch.equal(yn, rn)
    np.testing.assert_array_equal(bits(y)[~yn.numpy()], bits(ref)[~rn.numpy()])


@pytest.mark.parametrize("shape", [(2, 3, 8, 8), (1, 5, 7, 9), (3, 16, 36, 36)])
def test_backward_pass_matches_relu_and_pool_backward(shape):
    g = torch.Generator().manual_seed(7 + sum(shape))
    x = _special(shape, g)
    x = torch.nan_to_num(x.float(), nan=0.5).bfloat16()  # NaN windows: gradient routing is compared below
    r = torch.relu(x)
    gp = torch.randn(shape[0], shape[1], shape[2] // 2, shape[3] // 2, generator=g).bfloat16()
    # PyTorch: max_pool2d backward on the ReLU result, then threshold_backward
    rr = r.float().requires_grad_()
    torch.nn.functional.max_pool2d(rr, 2, 2).backward(gp.float())
    ref = torch.where(r.float() > 0, rr.grad, torch.zeros(())).bfloat16()
    rd = r.to(X)
    out = C().region_backward(rd, None, gp.to(X), rd, None, None, None, 0.0, None, list(shape))
    np.testing.assert_array_equal(bits(out), bits(ref))
    # same-shape gradient with a tap term and an extra term: one fp32 sum, one rounding
    gg = torch.randn(shape, generator=g).bfloat16()
    ta, tb, ex = (torch.randn(shape, generator=g).bfloat16() for _ in range(3))
    go = torch.tensor(0.75).to(X)
    out = C().region_backward(rd, gg.to(X), None, None, ex.to(X), ta.to(X), tb.to(X), 0.5, go, list(shape))
    v = gg.double() + ex.double() + 0.5 * 0.75 * (ta.double() - tb.double())
    ref = torch.where(r.double() > 0, v, torch.zeros((), dtype=torch.float64))
    got = out.cpu().double()
    ulp = torch.clamp(ref.abs(), min=2.0 ** -126) * 2.0 ** -8
    assert ((got - ref).abs() <= ulp + 1e-30).all()


def test_loss_partials_and_finish_against_float64():
    g = torch.Generator().manual_seed(11)
    a = torch.randn(40, 128, 18, 18, generator=g).bfloat16()
    b = torch.randn(40, 128, 18, 18, generator=g).bfloat16()
    P = C().region_loss_parts()
    part = torch.empty(2 * P, dtype=torch.float32, device=X)
    C().region_sqdiff(a.to(X), b.to(X), 0.25, part, 0)
    G = torch.randn(4, 64, 64, generator=g).bfloat16()
    T = torch.randn(1, 64, 64, generator=g).float()
    C().region_gram_sqdiff(G.to(X), T.to(X), 1296.0, 3.0, part, P)
    lf, lh = C().region_loss_finish(part)
    ref = 0.25 * ((a.double() - b.double()) ** 2).sum() + 3.0 * ((G.double() / 1296.0 - T.double()) ** 2).sum()
    assert abs(float(lf.cpu()) - float(ref)) <= 1e-5 * float(ref)
    assert abs(float(lh.cpu().float()) - float(ref)) <= 2.0 ** -8 * float(ref)
    # the same inputs give the same bits
    part2 = torch.empty(2 * P, dtype=torch.float32, device=X)
    C().region_sqdiff(a.to(X), b.to(X), 0.25, part2, 0)
    C().region_gram_sqdiff(G.to(X), T.to(X), 1296.0, 3.0, part2, P)
    assert torch.equal(part.cpu(), part2.cpu())


def test_gram_gradient_formula():
    g = torch.Generator().manual_seed(12)
    F = torch.randn(3, 32, 50, generator=g).bfloat16()
    G = (F.float() @ F.float().transpose(1, 2)).bfloat16()
    T = torch.randn(1, 32, 32, generator=g).float() * 10
    chw = 32.0 * 50
    S = C().region_gram_grad(G.to(X), T.to(X), chw, 0.01, torch.tensor(2.0).to(X))
    d = G.double() / chw - T.double()
    ref = 0.01 * 2.0 * (d + d.transpose(1, 2)) / chw
    got = S.cpu().double()
    assert ((got - ref).abs() <= ref.abs() * 2.0 ** -8 + 1e-30).all()
    assert torch.equal(S.cpu(), S.cpu().transpose(1, 2))


def vgg_layers(seed=0, widths=(3, 16, 16, 32, 32)):
    torch.manual_seed(seed)
    c = widths
    layers = [nn.Conv2d(c[0], c[1], 3, padding=1), nn.ReLU(), nn.Conv2d(c[1], c[2], 3, padding=1), nn.ReLU(),
              nn.MaxPool2d(2), nn.Conv2d(c[2], c[3], 3, padding=1), nn.ReLU(), nn.Conv2d(c[3], c[4], 3, padding=1),
              nn.ReLU(), nn.MaxPool2d(2), nn.Conv2d(c[4], c[4], 3, padding=1), nn.ReLU()]
    for m in layers:
        for p in m.parameters():
            p.requires_grad_(False)
    return [m.bfloat16() for m in layers]


def cpu_fp32_copy(layers):
    """The same layers in fp32 on the CPU (conv weights converted from bf16 exactly)."""
    out = []
    for m in layers:
        if isinstance(m, nn.Conv2d):
            n = nn.Conv2d(m.in_channels, m.out_channels, 3, padding=1)
            n.load_state_dict({k: v.float().cpu() for k, v in m.state_dict().items()})
            for p in n.parameters():
                p.requires_grad_(False)
        elif isinstance(m, nn.ReLU):
            n = nn.ReLU()
        else:
            n = nn.MaxPool2d(2)
        out.append(n)
    return out


def rel_l2(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).norm() / max(float(b.norm()), 1e-30))


def test_frozen_feature_mse_matches_eager_fp32():
    layers = vgg_layers()
    ref_layers = cpu_fp32_copy(layers)
    for m in layers:
        m.to(X)
    g = torch.Generator().manual_seed(5)
    x = torch.rand(4, 3, 20, 20, generator=g).bfloat16()
    t = torch.rand(4, 3, 20, 20, generator=g).bfloat16()
    taps = [3, 8, 11]
    chain = regions.FrozenFeatureChain.from_sequential(layers, taps)
    xd = x.to(X).requires_grad_()
    xdna_train.reset_mapped_cpu_stats()
    loss = regions.frozen_feature_mse(chain, xd, t.to(X))
    loss.backward()
    st = xdna_train.mapped_cpu_stats()
    for k in ("hip_region.conv_relu.run", "hip_region.maxpool2.run", "hip_region.sqdiff.run",
              "hip_region.backward.run"):
        assert st.get(k, {}).get("calls", 0) > 0, (k, st)
    assert loss.dtype == torch.bfloat16
    chain32 = regions.FrozenFeatureChain.from_sequential(ref_layers, taps)
    x32 = x.float().requires_grad_()
    ref = regions._eager_mse(chain32, x32, t.float())
    ref.backward()
    xe = x.to(X).requires_grad_()
    eager = regions._eager_mse(chain, xe, t.to(X))  # the eager bf16 ops on xdna
    eager.backward()
    e_loss = abs(float(loss.cpu().float()) - float(ref)) / abs(float(ref))
    e_eager = abs(float(eager.cpu().float()) - float(ref)) / abs(float(ref))
    g_reg, g_eager = rel_l2(xd.grad, x32.grad), rel_l2(xe.grad, x32.grad)
    print(f"loss vs fp32: region {e_loss:.3e}, eager bf16 {e_eager:.3e}; dX rel L2: region {g_reg:.3e}, "
          f"eager bf16 {g_eager:.3e}", flush=True)
    assert e_loss <= 1.5 * e_eager + 2.0 ** -8
    assert g_reg <= 1.5 * g_eager + 2.0 ** -8


def test_frozen_feature_loss_with_gram_terms_matches_eager_fp32():
    """The BASELINE style configuration's loss on its VGG19 prefix (through relu4_1) at its
    shapes: content MSE at relu2_2 against the content image's features, Gram terms at
    relu1_1 / 2_1 / 3_1 / 4_1 with weight 1e5, batch 40 of 36 x 36."""
    Generator, VGG = bench.style_models(torch, nn)
    torch.manual_seed(0)
    vgg = VGG().bfloat16()
    flat = []
    for layer in vgg.layers:
        flat += list(layer) if isinstance(layer, nn.Sequential) else [layer]
    for m in flat:
        for p in m.parameters():
            p.requires_grad_(False)
    names = ["conv1_1", "relu1_1", "conv1_2", "relu1_2", "pool1", "conv2_1", "relu2_1", "conv2_2", "relu2_2",
             "pool2", "conv3_1", "relu3_1", "conv3_2", "relu3_2", "conv3_3", "relu3_3", "conv3_4", "relu3_4",
             "pool3", "conv4_1", "relu4_1"]
    assert len(flat) == len(names)
    idx = {n: i for i, n in enumerate(names)}
    g = torch.Generator().manual_seed(9)
    x = torch.rand(40, 3, 36, 36, generator=g).bfloat16()
    content = torch.rand(40, 3, 36, 36, generator=g).bfloat16()
    style_img = torch.rand(1, 3, 36, 36, generator=g).bfloat16()
    ref_flat = cpu_fp32_copy(flat)
    style_taps = [idx[n] for n in ("relu1_1", "relu2_1", "relu3_1", "relu4_1")]
    # target Gram matrices from the fp32 chain (the same for both paths)
    with torch.no_grad():
        f = style_img.float()
        grams = {}
        for i, m in enumerate(ref_flat[: max(style_taps) + 1]):
            f = m(f)
            if i in style_taps:
                F3 = f.reshape(1, f.shape[1], -1)
                grams[i] = F3 @ F3.transpose(1, 2) / float(f[0].numel())
    taps = style_taps + [idx["relu2_2"]]
    for m in flat:
        m.to(X)
    chain = regions.FrozenFeatureChain.from_sequential(flat, taps)
    style = {k: (grams[k].to(X), 1e5) for k in style_taps}
    xd = x.to(X).requires_grad_()
    xdna_train.reset_mapped_cpu_stats()
    loss = regions.frozen_feature_loss(chain, xd, content.to(X), mse_taps=[idx["relu2_2"]], style=style)
    loss.backward()
    st = xdna_train.mapped_cpu_stats()
    for k in ("hip_region.conv_relu.run", "hip_region.gram_sqdiff.run", "hip_region.gram_grad.run",
              "hip_region.bmm.run"):
        assert st.get(k, {}).get("calls", 0) > 0, (k, st)
    assert loss.dtype == torch.float32
    chain32 = regions.FrozenFeatureChain.from_sequential(ref_flat, taps)
    x32 = x.float().requires_grad_()
    ref = regions._eager_loss(chain32, x32, content.float(), (idx["relu2_2"],),
                              {k: (v, 1e5) for k, v in grams.items()}, 1.0)
    ref.backward()
    # the eager bf16 ops on xdna (the backend's conv, relu, pool, bmm and fp32 losses): the
    # same rounding of the features, the error the region is held to
    xe = x.to(X).requires_grad_()
    eager = regions._eager_loss(chain, xe, content.to(X), (idx["relu2_2"],), style, 1.0)
    eager.backward()
    e_loss = abs(float(loss.cpu()) - float(ref)) / abs(float(ref))
    e_eager = abs(float(eager.cpu()) - float(ref)) / abs(float(ref))
    g_reg, g_eager = rel_l2(xd.grad, x32.grad), rel_l2(xe.grad, x32.grad)
    print(f"loss vs fp32: region {e_loss:.3e}, eager bf16 {e_eager:.3e}; dX rel L2: region {g_reg:.3e}, "
          f"eager bf16 {g_eager:.3e}", flush=True)
    assert e_loss <= 1.5 * e_eager + 2.0 ** -8
    assert g_reg <= 1.5 * g_eager + 2.0 ** -8


def test_fuse_perceptual_loss_pattern():
    """The reference's loss-module pattern: perceptual_vgg.model.features + feature_layers
    (+ use_norm / norm), compute_perceptual_loss routed through the region."""
    layers = vgg_layers(seed=1)

    class Norm(nn.Module):
        mean = [0.485, 0.456, 0.406]
        std = [0.229, 0.224, 0.225]

    class Net(nn.Module):
        def __init__(self):
            super().__init__()
            self.model = nn.Module()
            self.model.features = nn.Sequential(*layers)
            self.feature_layers = [3, 8]
            self.use_norm = True
            self.norm = Norm()

    class Loss(nn.Module):
        def __init__(self):
            super().__init__()
            self.perceptual_vgg = Net()

        def compute_perceptual_loss(self, input, target):
            raise AssertionError("the eager method must not run for eligible inputs")

    lm = Loss().to(X)
    assert regions.fuse_perceptual_loss(lm)
    g = torch.Generator().manual_seed(2)
    x = torch.rand(2, 3, 16, 16, generator=g).bfloat16().to(X).requires_grad_()
    t = torch.rand(2, 3, 16, 16, generator=g).bfloat16().to(X)
    loss = lm.compute_perceptual_loss(x, t)
    loss.backward()
    m = torch.tensor(Norm.mean).view(1, -1, 1, 1).bfloat16().to(X)
    s = torch.tensor(Norm.std).view(1, -1, 1, 1).bfloat16().to(X)
    chain = regions.FrozenFeatureChain.from_sequential(layers, [3, 8])
    x2 = x.detach().clone().requires_grad_()
    ref = regions.frozen_feature_mse(chain, (x2 - m) / s, (t - m) / s)
    ref.backward()
    assert torch.equal(loss.cpu(), ref.cpu())
    assert torch.equal(x.grad.cpu(), x2.grad.cpu())


def test_region_step_captured_and_replayed():
    layers = vgg_layers(seed=2)
    for m in layers:
        m.to(X)
    chain = regions.FrozenFeatureChain.from_sequential(layers, [3, 11])
    g = torch.Generator().manual_seed(4)
    x = torch.rand(2, 3, 16, 16, generator=g).bfloat16().to(X).requires_grad_()
    t = torch.rand(2, 3, 16, 16, generator=g).bfloat16().to(X)
    T = torch.rand(1, 32, 32, generator=g).to(X)

    def step():
        x.grad = None
        loss = regions.frozen_feature_loss(chain, x, t, mse_taps=[3], style={11: (T, 10.0)})
        loss.backward()
        return loss

    eager_loss = step().detach().cpu()
    eager_grad = x.grad.detach().cpu()
    gr = xdna_train.Graph()
    with xdna_train.graph(gr):
        gl = step()
    for _ in range(3):
        gr.replay()
        torch.xdna.synchronize()
        assert torch.equal(gl.detach().cpu(), eager_loss)
        assert torch.equal(x.grad.cpu(), eager_grad)
    gr.reset()
