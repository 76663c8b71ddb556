"""The fused norm + activation region on the GPU (the reference's fuse_norm_activation,
regions.py:426-546, with its CPU kernels region_kernels.cpp:346-457 as the contract):

* ReLU: forward output, running statistics and every gradient equal the unfused xdna pair
  (the same norm kernels, then relu / threshold_backward) bit for bit -- relu commutes
  with the one rounding, and the mask read from y is threshold_backward's.
* LeakyReLU: within rounding of an fp32 CPU reference, no further from it than the
  unfused bf16 pair (which rounds the norm output and the scaled gradient once more).
* The reference's pairing contract: the activation passes the fused output through once,
  deepcopy keeps a working pair, ineligible calls run both modules unchanged, and the
  region kernels ran (path counters).
"""
import copy

import numpy as np
import pytest
import torch
import torch.nn as nn

import xdna_train
from xdna_train import regions

pytestmark = pytest.mark.gpu
X = torch.device("xdna")


@pytest.fixture(scope="module", autouse=True)
def xdna():
    assert xdna_train.is_available(), "xdna device not available on the GPU box"
    xdna_train.set_npu_mode(2)
    return xdna_train


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy()


def rel_l2(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / max(float(b.norm()), 1e-30))


def make_norm(kind, c, seed, param_dtype=torch.bfloat16):
    torch.manual_seed(seed)
    m = nn.BatchNorm2d(c, momentum=0.2) if kind == "bn" else nn.InstanceNorm2d(c, affine=True)
    with torch.no_grad():
        m.weight.copy_(torch.rand(c) + 0.5)
        m.bias.copy_(torch.randn(c) * 0.3)
        if kind == "bn":
            m.running_mean.copy_(torch.randn(c) * 0.1)
            m.running_var.copy_(torch.rand(c) + 0.5)
    m = m.to(param_dtype)
    m.train()
    return m


def run_pair(norm, act, x, g):
    """y = act(norm(x)) and its gradients for the upstream gradient g."""
    xd = x.clone().requires_grad_()
    y = act(norm(xd))
    y.backward(g)
    return y.detach(), xd.grad, norm.weight.grad, norm.bias.grad


SHAPES = [(4, 32, 18, 18), (2, 64, 36, 36), (3, 8, 7, 9), (40, 128, 9, 9), (1, 16, 72, 72)]


@pytest.mark.parametrize("kind", ["bn", "in"])
@pytest.mark.parametrize("param_dtype", [torch.bfloat16, torch.float32])
def test_relu_pair_equals_unfused_bit_exact(kind, param_dtype):
    for i, shape in enumerate(SHAPES):
        gen = torch.Generator().manual_seed(10 + i)
        x = (torch.randn(*shape, generator=gen) * 2 + 0.5).bfloat16().to(X)
        g = torch.randn(*shape, generator=gen).bfloat16().to(X)
        ref_norm = make_norm(kind, shape[1], i, param_dtype).to(X)
        fused_norm = copy.deepcopy(ref_norm)
        act = nn.ReLU()
        assert regions.fuse_norm_activation(fused_norm, act)
        ref = run_pair(ref_norm, nn.ReLU(), x, g)
        xdna_train.reset_mapped_cpu_stats()
        got = run_pair(fused_norm, act, x, g)
        st = xdna_train.mapped_cpu_stats()
        key = "batch_norm_act" if kind == "bn" else "instance_norm_act"
        assert st.get(f"hip_region.{key}.run", {}).get("calls", 0) == 1, st
        assert st.get(f"hip_region.{key}_bwd.run", {}).get("calls", 0) == 1, st
        for name, a, b in zip(("y", "dx", "dweight", "dbias"), got, ref):
            np.testing.assert_array_equal(bits(a), bits(b), err_msg=f"{kind} {shape} {name}")
        if kind == "bn":
            for name in ("running_mean", "running_var", "num_batches_tracked"):
                np.testing.assert_array_equal(getattr(fused_norm, name).cpu().double().numpy(),
                                              getattr(ref_norm, name).cpu().double().numpy(), err_msg=f"{shape} {name}")


def cpu_reference(kind, norm, slope, x, g):
    """act(norm(x)) and its gradients in fp32 on the CPU (parameters from the bf16 ones)."""
    n32 = copy.deepcopy(norm).cpu().float()
    x32 = x.detach().cpu().float().requires_grad_()
    y = nn.functional.leaky_relu(n32(x32), slope)
    y.backward(g.detach().cpu().float())
    return y.detach(), x32.grad, n32.weight.grad, n32.bias.grad, n32


@pytest.mark.parametrize("kind", ["bn", "in"])
@pytest.mark.parametrize("slope", [0.2, 0.01, 0.0])
def test_leaky_pair_within_rounding_of_fp32(kind, slope):
    for i, shape in enumerate(SHAPES[:4]):
        gen = torch.Generator().manual_seed(30 + i)
        x = (torch.randn(*shape, generator=gen) * 2 + 0.5).bfloat16().to(X)
        g = torch.randn(*shape, generator=gen).bfloat16().to(X)
        base = make_norm(kind, shape[1], i).to(X)
        ref32 = cpu_reference(kind, base, slope, x, g)
        eager_norm, fused_norm = copy.deepcopy(base), copy.deepcopy(base)
        act = nn.LeakyReLU(slope)
        assert regions.fuse_norm_activation(fused_norm, act)
        eager = run_pair(eager_norm, nn.LeakyReLU(slope), x, g)
        xdna_train.reset_mapped_cpu_stats()
        got = run_pair(fused_norm, act, x, g)
        key = "batch_norm_act" if kind == "bn" else "instance_norm_act"
        assert xdna_train.mapped_cpu_stats().get(f"hip_region.{key}.run", {}).get("calls", 0) == 1
        for name, a, e, r in zip(("y", "dx", "dweight", "dbias"), got, eager, ref32):
            e_f, e_e = rel_l2(a, r), rel_l2(e, r)
            assert e_f <= 1.5 * e_e + 2.0 ** -8, (kind, shape, slope, name, e_f, e_e)
        # forward: within one bf16 ulp of the fp32 value (one rounding), beside an absolute
        # floor for the fp32 differences of the statistics where the output cancels to ~0
        yf, y32 = got[0].cpu().float(), ref32[0]
        tol = y32.abs() * 2.0 ** -7 + 1e-4 * float(y32.abs().max())
        assert bool(((yf - y32).abs() <= tol).all()), (kind, shape, slope)
        if kind == "bn":
            n32 = ref32[4]
            for name in ("running_mean", "running_var"):
                a = getattr(fused_norm, name).float().cpu()
                b = getattr(n32, name)
                assert rel_l2(a, b) <= 2.0 ** -7, (shape, name)


def test_nan_stays_in_its_plane():
    """A NaN input makes its instance-norm plane NaN forward and backward, as the unfused
    pair does, and leaves every other plane as the unfused pair computes it.  (The
    backward's NaN rule -- ReLU passes the gradient where y is NaN, as threshold_backward
    does; LeakyReLU scales it -- only meets planes that are NaN throughout.)"""
    shape = (2, 4, 6, 6)
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(*shape, generator=gen).bfloat16()
    x[0, 1, 2, 3] = float("nan")
    x = x.to(X)
    g = torch.randn(*shape, generator=gen).bfloat16().to(X)
    for act_cls in (nn.ReLU, lambda: nn.LeakyReLU(0.2)):
        ref_norm = make_norm("in", 4, 0).to(X)
        fused_norm = copy.deepcopy(ref_norm)
        act = act_cls()
        assert regions.fuse_norm_activation(fused_norm, act)
        ref = run_pair(ref_norm, act_cls(), x, g)
        got = run_pair(fused_norm, act, x, g)
        # the plane holding the NaN is NaN throughout, others are finite and equal
        ok = torch.ones(shape, dtype=torch.bool)
        ok[0, 1] = False
        for name, a, b in zip(("y", "dx"), got[:2], ref[:2]):
            a, b = a.cpu().float(), b.cpu().float()
            assert torch.isnan(a[~ok]).all() and torch.isnan(b[~ok]).all(), name
            if act_cls is nn.ReLU:
                np.testing.assert_array_equal(bits(a[ok]), bits(b[ok]), err_msg=name)
            else:
                assert rel_l2(a[ok], b[ok]) <= 2.0 ** -7, name


def test_pairing_contract():
    shape = (2, 8, 12, 12)
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(*shape, generator=gen).bfloat16().to(X)
    norm = make_norm("bn", 8, 1).to(X)
    act = nn.LeakyReLU(0.1)
    assert regions.fuse_norm_activation(norm, act)
    assert regions.fuse_norm_activation(norm, act)  # already paired with it
    assert not regions.fuse_norm_activation(norm, nn.ReLU())  # paired with another
    assert not regions.fuse_norm_activation(nn.BatchNorm2d(4), nn.Sigmoid())
    assert not regions.fuse_norm_activation(nn.LayerNorm(4), nn.ReLU())
    y = norm(x)
    assert regions.awaits_activation(y, act)
    z = act(y)
    assert z is y  # passed through once
    w = act(y)  # a second call activates
    np.testing.assert_array_equal(bits(w), bits(nn.functional.leaky_relu(y, 0.1)))
    # the slope is read at call time
    act.negative_slope = 0.3
    y2 = norm(x)
    ref = nn.functional.leaky_relu(nn.BatchNorm2d.forward(norm, x), 0.3)
    assert rel_l2(act(y2), ref) <= 2.0 ** -7
    # a negative slope runs both modules unchanged (the output's sign no longer masks)
    act.negative_slope = -0.5
    y3 = norm(x)
    assert not regions.awaits_activation(y3, act)
    # eval mode and CPU tensors: eager
    norm.eval()
    assert not regions.awaits_activation(norm(x), act)
    norm.train()
    cpu_norm = make_norm("bn", 8, 1)
    cpu_act = nn.ReLU()
    assert regions.fuse_norm_activation(cpu_norm, cpu_act)
    yc = cpu_act(cpu_norm(x.cpu()))
    assert not regions.awaits_activation(yc, cpu_act) and bool((yc >= 0).all())


def test_deepcopy_keeps_a_working_pair():
    model = nn.Sequential(nn.Conv2d(4, 8, 3, padding=1), nn.InstanceNorm2d(8, affine=True), nn.ReLU(),
                          nn.Conv2d(8, 8, 3, padding=1), nn.BatchNorm2d(8), nn.LeakyReLU(0.2)).bfloat16().to(X)
    assert regions.fuse_norm_activations(model) == 2
    clone = copy.deepcopy(model)
    assert regions.paired_activation(clone[1]) is clone[2] and regions.paired_activation(clone[4]) is clone[5]
    assert clone[1].forward.norm is clone[1]
    gen = torch.Generator().manual_seed(4)
    x = torch.randn(2, 4, 16, 16, generator=gen).bfloat16().to(X)
    xdna_train.reset_mapped_cpu_stats()
    y = clone(x)
    st = xdna_train.mapped_cpu_stats()
    assert st.get("hip_region.instance_norm_act.run", {}).get("calls", 0) == 1
    assert st.get("hip_region.batch_norm_act.run", {}).get("calls", 0) == 1
    plain = copy.deepcopy(model)
    for m in plain.modules():
        regions.unfuse_norm_activation(m)
        m.__dict__.pop("forward", None)  # the activations' guards
    ref = plain(x)
    assert rel_l2(y, ref) <= 2.0 ** -7


def test_style_generator_step_with_fused_pairs():
    """The BASELINE style generator with its norm + ReLU pairs fused: one training step's
    loss and parameter gradients against the same step unfused (ReLU pairs are bit-exact
    per op; the step's other ops are shared)."""
    import bench
    Generator, _ = bench.style_models(torch, nn)
    torch.manual_seed(0)
    gen_a = Generator().bfloat16().to(X)
    gen_b = copy.deepcopy(gen_a)
    n = regions.fuse_norm_activations(gen_b)
    assert n == 10, n  # 3 downsampling blocks, the first block of 5 residual bodies, 2 upsampling blocks
    g = torch.Generator().manual_seed(1)
    x = torch.rand(4, 3, 36, 36, generator=g).bfloat16().to(X)
    grads = []
    for m in (gen_a, gen_b):
        y = m(x)
        (y.float() ** 2).mean().backward()
        grads.append((y.detach(), [p.grad for p in m.parameters()]))
    np.testing.assert_array_equal(bits(grads[0][0]), bits(grads[1][0]))
    for a, b in zip(grads[0][1], grads[1][1]):
        np.testing.assert_array_equal(bits(a), bits(b))
