"""The region module's host logic without a GPU: which layer chains a frozen-feature
region accepts (plain Conv2d / ReLU / MaxPool2d(2, 2), frozen weights, a conv first; the
reference's rules, regions.py:137-195), which convs fuse their ReLU, and the switch."""
import torch
import torch.nn as nn

from xdna_train import regions


def vgg_block():
    return [nn.Conv2d(3, 8, 3, padding=1), nn.ReLU(), nn.Conv2d(8, 8, 3, padding=1), nn.ReLU(),
            nn.MaxPool2d(2), nn.Conv2d(8, 16, 3, padding=1), nn.ReLU()]


def frozen(layers):
    for m in layers:
        for p in m.parameters():
            p.requires_grad_(False)
    return layers


def test_chain_parses_and_fuses_relus():
    layers = frozen(vgg_block())
    chain = regions.FrozenFeatureChain.from_sequential(layers, [3, 6])
    assert chain is not None and chain.taps == (3, 6)
    assert chain.kinds == ("conv", "relu", "conv", "relu", "maxpool2", "conv", "relu")
    assert chain.fused_relu == (True, False, True, False, False, True, False)
    assert chain.current()


def test_tapped_conv_output_is_not_fused():
    chain = regions.FrozenFeatureChain.from_sequential(frozen(vgg_block()), [2, 3])
    assert chain.fused_relu[:4] == (True, False, False, False)


def test_rejected_chains():
    assert regions.FrozenFeatureChain.from_sequential(vgg_block(), [3]) is None  # trainable weights
    layers = frozen(vgg_block())
    layers[1] = nn.LeakyReLU()
    assert regions.FrozenFeatureChain.from_sequential(layers, [3]) is None
    layers = frozen(vgg_block())
    layers[4] = nn.MaxPool2d(3)
    assert regions.FrozenFeatureChain.from_sequential(layers, [6]) is None
    layers = frozen(vgg_block())
    assert regions.FrozenFeatureChain.from_sequential(layers[1:], [2]) is None  # first layer not a conv
    assert regions.FrozenFeatureChain.from_sequential(frozen(vgg_block()), []) is None
    assert regions.FrozenFeatureChain.from_sequential(frozen(vgg_block()), [7]) is None
    layers = frozen(vgg_block())
    layers[2].register_forward_hook(lambda *a: None)
    assert regions.FrozenFeatureChain.from_sequential(layers, [3]) is None


def test_model_surgery_makes_the_chain_stale():
    layers = frozen(vgg_block())
    chain = regions.FrozenFeatureChain.from_sequential(layers, [3])
    layers[2].stride = (2, 2)
    assert not chain.current()


def test_cpu_tensors_are_not_eligible_and_switch(monkeypatch):
    chain = regions.FrozenFeatureChain.from_sequential(frozen(vgg_block()), [3])
    x = torch.rand(1, 3, 8, 8).bfloat16().requires_grad_()
    assert not chain.eligible(x, torch.rand(1, 3, 8, 8).bfloat16())
    monkeypatch.setenv("XDNA_REGIONS", "0")
    assert not regions.enabled()


def test_eager_paths_on_cpu_match_the_definition():
    """Ineligible inputs (CPU tensors) take the eager ops: the MSE over concatenated taps
    and the Gram style terms, as written out here."""
    torch.manual_seed(0)
    layers = frozen(vgg_block())
    chain = regions.FrozenFeatureChain.from_sequential(layers, [3, 6])
    x = torch.rand(2, 3, 8, 8, requires_grad=True)
    t = torch.rand(2, 3, 8, 8)
    loss = regions.frozen_feature_mse(chain, x, t)
    f = [x]
    for m in layers:
        f.append(m(f[-1]))
    g = [t]
    for m in layers:
        g.append(m(g[-1]))
    a = torch.cat([f[4].reshape(-1), f[7].reshape(-1)])
    b = torch.cat([g[4].reshape(-1), g[7].reshape(-1)])
    assert torch.allclose(loss, ((a - b) ** 2).mean())
    T = torch.rand(1, 16, 16)
    loss2 = regions.frozen_feature_loss(chain, x, t, mse_taps=[3], style={6: (T, 3.0)})
    F3 = f[7].reshape(2, 16, -1)
    gram = F3 @ F3.transpose(1, 2) / (16 * 4 * 4)
    ref = ((f[4] - g[4]) ** 2).mean() + 3.0 * ((gram - T) ** 2).mean()
    assert torch.allclose(loss2, ref, rtol=1e-5)


def test_norm_activation_pairing_on_the_cpu():
    """fuse_norm_activation's pairing rules (the reference's, regions.py:521-546, widened to
    InstanceNorm2d); on CPU tensors the pair runs both modules unchanged."""
    import copy

    import bench
    bn, act = nn.BatchNorm2d(4), nn.LeakyReLU(0.2)
    assert regions.fuse_norm_activation(bn, act)
    assert regions.fuse_norm_activation(bn, act)
    assert not regions.fuse_norm_activation(bn, nn.ReLU())
    assert not regions.fuse_norm_activation(nn.BatchNorm2d(4), nn.Sigmoid())
    assert not regions.fuse_norm_activation(nn.BatchNorm1d(4), nn.ReLU())
    assert not regions.fuse_norm_activation(nn.InstanceNorm2d(4), nn.GELU())
    assert regions.paired_activation(bn) is act and not list(bn.children())
    assert set(bn.state_dict()) == set(nn.BatchNorm2d(4).state_dict())
    torch.manual_seed(0)
    x = torch.randn(2, 4, 5, 5)
    ref_bn = nn.BatchNorm2d(4)
    y = act(bn(x))
    ref = nn.functional.leaky_relu(ref_bn(x), 0.2)
    assert torch.equal(y, ref) and not regions.awaits_activation(y, act)
    assert torch.equal(bn.running_mean, ref_bn.running_mean) and int(bn.num_batches_tracked) == 1
    clone = copy.deepcopy(nn.Sequential(bn, act))
    assert regions.paired_activation(clone[0]) is clone[1] and clone[0].forward.norm is clone[0]
    regions.unfuse_norm_activation(clone[0])
    assert regions.paired_activation(clone[0]) is None and regions.paired_activation(bn) is act
    Generator, _ = bench.style_models(torch, nn)
    assert regions.fuse_norm_activations(Generator()) == 10


def test_norm_activation_switch(monkeypatch):
    monkeypatch.setenv("XDNA_REGIONS", "0")
    assert not regions.fuse_norm_activation(nn.BatchNorm2d(4), nn.ReLU())


def test_perceptual_route_on_the_cpu():
    """fuse_perceptual_loss on the loss-module pattern: the route re-parses after model
    surgery, follows a deepcopy to the copy's own layers, and runs the module's own method
    for inputs the region does not take (CPU tensors here)."""
    import copy

    class Norm(nn.Module):
        mean = [0.5, 0.4, 0.3]
        std = [0.2, 0.25, 0.3]

    class Net(nn.Module):
        def __init__(self):
            super().__init__()
            self.model = nn.Module()
            self.model.features = nn.Sequential(*frozen(vgg_block()))
            self.feature_layers = [3, 6]
            self.use_norm = True
            self.norm = Norm()

    class Loss(nn.Module):
        def __init__(self):
            super().__init__()
            self.perceptual_vgg = Net()
            self.own_calls = 0

        def compute_perceptual_loss(self, input, target):
            self.own_calls += 1
            f = self.perceptual_vgg.model.features
            return ((f(input) - f(target)) ** 2).mean()

    lm = Loss()
    assert regions.perceptual_route(lm) is None
    assert regions.fuse_perceptual_loss(lm)
    route = regions.perceptual_route(lm)
    assert route is not None and route.owner is lm
    chain = route.chain()
    assert chain.taps == (3, 6) and chain.layers == list(lm.perceptual_vgg.model.features)
    assert route.chain() is chain  # cached while nothing changes
    x, t = torch.rand(1, 3, 8, 8), torch.rand(1, 3, 8, 8)
    got = lm.compute_perceptual_loss(x, t)
    assert lm.own_calls == 1 and torch.equal(got, Loss.compute_perceptual_loss(lm, x, t))
    clone = copy.deepcopy(lm)
    croute = regions.perceptual_route(clone)
    assert croute.owner is clone and croute.chain().layers == list(clone.perceptual_vgg.model.features)
    lm.perceptual_vgg.model.features[2].stride = (2, 2)  # surgery: parsed again
    strided = route.chain()
    assert strided is not chain and strided.fused_relu[2] is False and strided.current()
    handle = lm.perceptual_vgg.model.features[5].register_forward_hook(lambda *a: None)
    assert route.chain() is None  # a hooked layer: the module's own method runs
    handle.remove()
    assert route.chain() is not None
    lm.perceptual_vgg.feature_layers = [1]
    assert route.chain().taps == (1,)
    # patterns the region cannot take are not installed
    bad = Loss()
    bad.perceptual_vgg.model.features[0].weight.requires_grad_(True)
    assert not regions.fuse_perceptual_loss(bad) and regions.perceptual_route(bad) is None
    nonorm = Loss()
    nonorm.perceptual_vgg.norm = nn.Module()
    assert not regions.fuse_perceptual_loss(nonorm)
