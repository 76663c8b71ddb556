"""mse_loss / mse_loss_backward and the 2x2 max-pool on their HIP kernels (csrc/loss.hip,
csrc/region.hip) through the aten ops a plain training script calls.

* mse_loss (mean and sum; fp32 and bf16; same-shape targets and targets broadcast over the
  batch, as a style loss's ``T.expand_as(G)``; vector and element paths): the forward
  against a float64 sum of the same operands (fp32 within 1e-6 relative, bf16 within one
  rounding), bit-identical across repeated calls (fixed partition, fixed order whichever
  workgroup finishes last); the backward against 2 / n * (a - b) * go in float64, within
  one rounding of the operands' dtype; reduction 'none' keeps PyTorch-ROCm's kernel.
* max_pool2d (kernel 2, stride 2, floor mode): output and input gradient bit-exact with
  PyTorch's CPU kernel on the same bf16 values (odd sizes included), counters show the HIP
  kernels ran; other pools keep PyTorch's composite.
* a captured step of both, replayed with eager work between replays, equals the eager step.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import xdna_train

pytestmark = pytest.mark.gpu
X = torch.device("xdna")


@pytest.fixture(scope="module", autouse=True)
def xdna():
    assert xdna_train.is_available(), "xdna device not available on the GPU box"
    xdna_train.set_npu_mode(2)
    return xdna_train


def _calls(name):
    return xdna_train.mapped_cpu_stats().get(name, {}).get("calls", 0)


def _bits(t):
    t = t.detach().cpu().contiguous()
    return t.view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32).numpy()


CASES = [  # (input shape, target shape to expand, dtype)
    ((40, 64, 64), None, torch.float32),           # Gram-like, vector path
    ((40, 64, 64), (1, 64, 64), torch.float32),    # broadcast target (period 4096)
    ((8, 128, 18, 18), None, torch.bfloat16),      # feature taps, vector path
    ((7, 3, 5, 3), None, torch.float32),           # odd sizes: element path
    ((6, 33, 7), (1, 33, 7), torch.bfloat16),      # broadcast with an odd period
    ((3, 1000003 // 3), None, torch.float32),      # long, odd
]


@pytest.mark.parametrize("shape,tshape,dtype", CASES)
@pytest.mark.parametrize("reduction", ["mean", "sum"])
def test_mse_loss_forward_and_backward(shape, tshape, dtype, reduction):
    g = torch.Generator().manual_seed(sum(shape) + len(reduction))
    a = torch.randn(*shape, generator=g).to(dtype)
    t = torch.randn(*(tshape or shape), generator=g).to(dtype)
    te = t.expand(*shape)
    n = a.numel()
    fwd0, bwd0 = _calls("hip_mse_loss.fwd.run"), _calls("hip_mse_loss.bwd.run")
    ad = a.to(X).requires_grad_()
    td = t.to(X).expand(*shape)
    loss = F.mse_loss(ad, td, reduction=reduction)
    go = torch.tensor(0.75, dtype=dtype)
    loss.backward(go.to(X))
    assert _calls("hip_mse_loss.fwd.run") == fwd0 + 1 and _calls("hip_mse_loss.bwd.run") == bwd0 + 1
    assert loss.dtype == dtype and loss.shape == ()
    d = a.double() - te.double()
    ref = (d * d).sum() / (n if reduction == "mean" else 1)
    got = float(loss.detach().cpu().double())
    tol = 1e-6 if dtype == torch.float32 else 2.0 ** -8
    assert abs(got - float(ref)) <= tol * abs(float(ref)), (got, float(ref))
    # the same bits on every call
    for _ in range(3):
        again = F.mse_loss(a.to(X), td, reduction=reduction)
        assert np.array_equal(_bits(again), _bits(loss))
    norm = 2.0 / n if reduction == "mean" else 2.0
    gref = (norm * d * float(go)).numpy()
    gg = ad.grad.detach().cpu().double().numpy()
    err = np.abs(gg - gref)
    ulp = np.maximum(np.abs(gref), 1e-30) * (2.0 ** -23 if dtype == torch.float32 else 2.0 ** -8)
    # fp32: three roundings (difference, two products); bf16: those plus the final rounding
    assert (err <= 8 * ulp + 1e-30).all(), float((err / ulp).max())


def test_mse_loss_target_gradient_and_none():
    g = torch.Generator().manual_seed(3)
    a = torch.randn(4, 5, 6, generator=g)
    t = torch.randn(4, 5, 6, generator=g)
    ad, td = a.to(X).requires_grad_(), t.to(X).requires_grad_()
    F.mse_loss(ad, td).backward()
    ac, tc = a.clone().requires_grad_(), t.clone().requires_grad_()
    F.mse_loss(ac, tc).backward()
    torch.testing.assert_close(ad.grad.cpu(), ac.grad, rtol=1e-6, atol=1e-7)
    torch.testing.assert_close(td.grad.cpu(), tc.grad, rtol=1e-6, atol=1e-7)
    rocm0 = _calls("aten::mse_loss.rocm")
    out = F.mse_loss(a.to(X), t.to(X), reduction="none")
    assert _calls("aten::mse_loss.rocm") == rocm0 + 1
    torch.testing.assert_close(out.cpu(), F.mse_loss(a, t, reduction="none"))


@pytest.mark.parametrize("shape", [(40, 64, 36, 36), (4, 8, 9, 9), (2, 3, 7, 10), (1, 2, 2, 2)])
def test_max_pool2d_bit_exact(shape):
    g = torch.Generator().manual_seed(sum(shape))
    x = torch.randn(*shape, generator=g).bfloat16()
    x[0, 0, 0, :2] = x[0, 0, 1, 0]  # ties: the first maximum in row-major order wins
    dy = torch.randn(shape[0], shape[1], shape[2] // 2, shape[3] // 2, generator=g).bfloat16()
    f0, b0 = _calls("hip_maxpool2.fwd.run"), _calls("hip_maxpool2.bwd.run")
    xd = x.to(X).requires_grad_()
    y = F.max_pool2d(xd, 2)
    y.backward(dy.to(X))
    assert _calls("hip_maxpool2.fwd.run") == f0 + 1 and _calls("hip_maxpool2.bwd.run") == b0 + 1
    xc = x.clone().requires_grad_()
    yc = F.max_pool2d(xc, 2)
    yc.backward(dy)
    assert np.array_equal(_bits(y), _bits(yc))
    assert np.array_equal(_bits(xd.grad), _bits(xc.grad))


def test_other_pools_keep_the_composite():
    x = torch.randn(2, 3, 9, 9).bfloat16()
    f0 = _calls("hip_maxpool2.fwd.run")
    for kw in ({"kernel_size": 3, "stride": 2}, {"kernel_size": 2, "stride": 2, "ceil_mode": True},
               {"kernel_size": 2, "stride": 1}, {"kernel_size": 2, "padding": 1}):
        y = F.max_pool2d(x.to(X), **kw)
        assert torch.equal(y.cpu(), F.max_pool2d(x, **kw)), kw
    assert _calls("hip_maxpool2.fwd.run") == f0
    y, idx = F.max_pool2d(x.to(X), 2, return_indices=True)
    yc, ic = F.max_pool2d(x, 2, return_indices=True)
    assert torch.equal(y.cpu(), yc) and torch.equal(idx.cpu(), ic)


def test_captured_loss_step_matches_eager():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(8, 16, 12, 12, generator=g).bfloat16().to(X)
    t = torch.randn(1, 16, 6, 6, generator=g).bfloat16().to(X)
    w = torch.randn(8, 16, 6, 6, generator=g).bfloat16().to(X).requires_grad_()

    def step():
        w.grad = None
        p = F.max_pool2d(x * w.repeat_interleave(2, 2).repeat_interleave(2, 3), 2)
        loss = F.mse_loss(p.float(), t.float().expand_as(p)) + 0.5 * F.mse_loss(p, t.expand_as(p)).float()
        loss.backward()
        return loss

    eager_loss = _bits(step())
    eager_grad = _bits(w.grad)
    graph = torch.xdna.Graph()
    with torch.xdna.graph(graph):
        gl = step()
    for _ in range(3):
        junk = torch.randn(1000, device=X)
        _ = F.mse_loss(junk, junk * 2)
        graph.replay()
        torch.xdna.synchronize()
        assert np.array_equal(_bits(gl), eager_loss)
        assert np.array_equal(_bits(w.grad), eager_grad)
    graph.reset()
