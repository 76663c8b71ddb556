"""InstanceNorm on the xdna device: the HIP instance-norm kernels (the backend's
instance_norm override at the autograd level) and the HIP batch-norm kernels (reached
through native_batch_norm / native_batch_norm_backward, by batch_norm and by the
instance_norm forms the override leaves to PyTorch's composite) against an fp64 autograd
reference computed from the same bf16 inputs on the CPU.
Tolerance: bf16 outputs within 2 bf16 ulp (floor at 2^-8 of the largest magnitude) and
relative L2 <= 1e-2; parameter gradients within 2 bf16 ulp (bf16 parameters: one
rounding of an fp32 sum) or 1e-4 relative (fp32 parameters)."""
import numpy as np
import pytest
import torch

import oracle
import xdna_train
from gpu_util import check_bf16

pytestmark = pytest.mark.gpu
X = torch.device("xdna")


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("shape,affine,pdtype", [
    ((40, 128, 9, 9), True, torch.bfloat16),
    ((40, 32, 36, 36), True, torch.bfloat16),
    ((2, 3, 5, 7), False, torch.bfloat16),
    ((3, 5, 1, 2), True, torch.float32),
    ((1, 4, 130, 130), True, torch.bfloat16),
])
def test_instance_norm_matches_fp64(shape, affine, pdtype):
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(shape, generator=g) * 3 + 0.5).bfloat16()
    dy = torch.randn(shape, generator=g).bfloat16()
    C = shape[1]
    w = (torch.rand(C, generator=g) + 0.5).to(pdtype) if affine else None
    b = (torch.randn(C, generator=g) * 0.1).to(pdtype) if affine else None
    # reference: fp64 instance norm of the bf16 inputs
    xr = x.double().requires_grad_(True)
    wr = w.double().requires_grad_(True) if affine else None
    br = b.double().requires_grad_(True) if affine else None
    yr = torch.nn.functional.instance_norm(xr, weight=wr, bias=br, eps=1e-5)
    yr.backward(dy.double())
    # device
    xd = x.to(X).requires_grad_(True)
    wd = w.to(X).requires_grad_(True) if affine else None
    bd = b.to(X).requires_grad_(True) if affine else None
    xdna_train.reset_mapped_cpu_stats()
    yd = torch.nn.functional.instance_norm(xd, weight=wd, bias=bd, eps=1e-5)
    yd.backward(dy.to(X))
    torch.xdna.synchronize()
    stats = xdna_train.mapped_cpu_stats()
    # affine norms take the instance-norm kernels, the others PyTorch's composite over
    # the batch-norm kernels
    kind = "hip_instance_norm" if affine else "hip_batch_norm"
    assert stats.get(f"{kind}.fwd.run", {}).get("calls", 0) == 1, stats
    assert stats.get(f"{kind}.bwd.run", {}).get("calls", 0) == 1, stats
    assert "aten::native_batch_norm.rocm" not in stats, stats
    check_bf16(bits(yd), yr.detach().numpy(), what="instance_norm out")
    check_bf16(bits(xd.grad), xr.grad.numpy(), what="instance_norm dx")
    if affine:
        assert wd.grad.dtype == pdtype and bd.grad.dtype == pdtype
        check_param_grads(((wd.grad, wr.grad, "dweight"), (bd.grad, br.grad, "dbias")), pdtype)


def check_param_grads(pairs, pdtype):
    for got, ref, name in pairs:
        gv = got.detach().cpu().double().numpy()
        rv = ref.numpy()
        if pdtype == torch.bfloat16:
            tol = 2 * oracle.bf16_ulp(np.abs(rv) + np.abs(rv).max() * 2.0 ** -8)
        else:
            tol = 1e-4 * (np.abs(rv) + np.abs(rv).max())
        assert (np.abs(gv - rv) <= tol).all(), (name, np.abs(gv - rv).max(), tol.max())


@pytest.mark.parametrize("need", ["x", "params"])
def test_instance_norm_partial_grads(need):
    """Only the input, or only the parameters, require gradients."""
    g = torch.Generator().manual_seed(11)
    shape = (6, 24, 10, 11)
    x = torch.randn(shape, generator=g).bfloat16()
    dy = torch.randn(shape, generator=g).bfloat16()
    w = (torch.rand(24, generator=g) + 0.5).bfloat16()
    b = torch.randn(24, generator=g).bfloat16()
    xr = x.double().requires_grad_(need == "x")
    wr = w.double().requires_grad_(need == "params")
    br = b.double().requires_grad_(need == "params")
    torch.nn.functional.instance_norm(xr, weight=wr, bias=br).backward(dy.double())
    xd = x.to(X).requires_grad_(need == "x")
    wd = w.to(X).requires_grad_(need == "params")
    bd = b.to(X).requires_grad_(need == "params")
    xdna_train.reset_mapped_cpu_stats()
    torch.nn.functional.instance_norm(xd, weight=wd, bias=bd).backward(dy.to(X))
    torch.xdna.synchronize()
    stats = xdna_train.mapped_cpu_stats()
    assert stats.get("hip_instance_norm.bwd.run", {}).get("calls", 0) == 1, stats
    if need == "x":
        assert wd.grad is None and bd.grad is None
        check_bf16(bits(xd.grad), xr.grad.numpy(), what="instance_norm dx")
    else:
        assert xd.grad is None
        check_param_grads(((wd.grad, wr.grad, "dweight"), (bd.grad, br.grad, "dbias")), torch.bfloat16)


def test_instance_norm_module_channels_last_and_no_grad():
    """nn.InstanceNorm2d(affine) on a channels-last input, then under no_grad."""
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 16, 9, 13, generator=g).bfloat16()
    m = torch.nn.InstanceNorm2d(16, affine=True).bfloat16()
    with torch.no_grad():
        m.weight.copy_(torch.rand(16, generator=g) + 0.5)
        m.bias.copy_(torch.randn(16, generator=g))
    ref = torch.nn.functional.instance_norm(x.double(), weight=m.weight.double(), bias=m.bias.double())
    md = m.to(X)
    xd = x.to(X).contiguous(memory_format=torch.channels_last)
    y = md(xd)
    check_bf16(bits(y), ref.detach().numpy(), what="channels-last instance_norm out")
    with torch.no_grad():
        y2 = md(x.to(X))
    assert y2.grad_fn is None
    check_bf16(bits(y2), ref.detach().numpy(), what="no_grad instance_norm out")


def test_instance_norm_lone_weight_uses_batch_norm_kernels():
    """A weight without a bias leaves instance_norm to PyTorch's composite, whose
    native_batch_norm calls still reach the HIP batch-norm kernels."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 8, 7, 7, generator=g).bfloat16()
    w = (torch.rand(8, generator=g) + 0.5).bfloat16()
    ref = torch.nn.functional.instance_norm(x.double(), weight=w.double())
    xdna_train.reset_mapped_cpu_stats()
    y = torch.nn.functional.instance_norm(x.to(X), weight=w.to(X))
    torch.xdna.synchronize()
    stats = xdna_train.mapped_cpu_stats()
    assert "hip_instance_norm.fwd.run" not in stats, stats
    assert stats.get("hip_batch_norm.fwd.run", {}).get("calls", 0) == 1, stats
    check_bf16(bits(y), ref.numpy(), what="composite instance_norm out")


@pytest.mark.parametrize("pdtype", [torch.bfloat16, torch.float32])
def test_batch_norm_training_without_running_stats(pdtype):
    g = torch.Generator().manual_seed(9)
    shape = (5, 12, 6, 7)
    x = (torch.randn(shape, generator=g) * 2 - 1).bfloat16()
    dy = torch.randn(shape, generator=g).bfloat16()
    w = (torch.rand(12, generator=g) + 0.5).to(pdtype)
    b = torch.randn(12, generator=g).to(pdtype)
    xr, wr, br = (t.double().requires_grad_(True) for t in (x, w, b))
    torch.nn.functional.batch_norm(xr, None, None, wr, br, training=True).backward(dy.double())
    xd, wd, bd = (t.to(X).requires_grad_(True) for t in (x, w, b))
    xdna_train.reset_mapped_cpu_stats()
    yd = torch.nn.functional.batch_norm(xd, None, None, wd, bd, training=True)
    yd.backward(dy.to(X))
    torch.xdna.synchronize()
    stats = xdna_train.mapped_cpu_stats()
    assert stats.get("hip_batch_norm.fwd.run", {}).get("calls", 0) == 1, stats
    assert stats.get("hip_batch_norm.bwd.run", {}).get("calls", 0) == 1, stats
    check_bf16(bits(xd.grad), xr.grad.numpy(), what="batch_norm dx")
    check_param_grads(((wd.grad, wr.grad, "dweight"), (bd.grad, br.grad, "dbias")), pdtype)


def test_batch_norm_running_stats_training_on_hip_eval_on_rocm():
    """Training mode with running statistics takes the spatial HIP kernels; eval mode
    (normalising by the running statistics) is served by PyTorch-ROCm on aliases."""
    x = torch.randn(4, 8, 6, 6).bfloat16()
    bn = torch.nn.BatchNorm2d(8).bfloat16()
    ref = bn(x.clone())
    bnd = torch.nn.BatchNorm2d(8).bfloat16().to(X)
    xdna_train.reset_mapped_cpu_stats()
    out = bnd(x.to(X))
    torch.xdna.synchronize()
    stats = xdna_train.mapped_cpu_stats()
    assert stats.get("hip_batch_norm_train.fwd.run", {}).get("calls", 0) == 1, stats
    assert torch.allclose(out.cpu().float(), ref.float(), atol=3e-2, rtol=3e-2)
    assert torch.allclose(bnd.running_mean.cpu().float(), bn.running_mean.float(), atol=1e-2)
    bn.eval()
    bnd.eval()
    xdna_train.reset_mapped_cpu_stats()
    out = bnd(x.to(X))
    stats = xdna_train.mapped_cpu_stats()
    assert stats.get("aten::native_batch_norm.rocm", {}).get("calls", 0) >= 1, stats
    assert torch.allclose(out.cpu().float(), bn(x.clone()).float(), atol=3e-2, rtol=3e-2)


@pytest.mark.parametrize("shape,track", [
    ((128, 64, 64, 64), True),   # config 5's first stage: 524288 elements per channel
    ((128, 512, 8, 8), True),
    ((16, 32, 9, 9), True),      # short channels, running statistics
    ((3, 5, 7, 5), True),        # planes not a multiple of 8 (element path)
    ((4, 48, 200, 100), False),  # long channels, no running statistics
])
def test_batch_norm_training_matches_fp64(shape, track):
    """BatchNorm2d in training mode with running statistics (bf16 module): the spatial
    batch-norm kernels against fp64 batch_norm of the same bf16 inputs; running mean and
    variance (momentum 0.1, unbiased variance) within 1 bf16 ulp of the fp64 update."""
    print("batch norm", shape, track, flush=True)
    g = torch.Generator().manual_seed(11)
    C = shape[1]
    x = (torch.randn(shape, generator=g) * 2 + 0.7).bfloat16()
    dy = torch.randn(shape, generator=g).bfloat16()
    w = (torch.rand(C, generator=g) + 0.5).bfloat16()
    b = (torch.randn(C, generator=g) * 0.1).bfloat16()
    rm0 = (torch.randn(C, generator=g) * 0.1).bfloat16()
    rv0 = (torch.rand(C, generator=g) + 0.5).bfloat16()
    # reference in fp64
    xr = x.double().requires_grad_(True)
    wr = w.double().requires_grad_(True)
    br = b.double().requires_grad_(True)
    rmr, rvr = rm0.double().clone(), rv0.double().clone()
    yr = torch.nn.functional.batch_norm(xr, rmr if track else None, rvr if track else None, wr, br,
                                        training=True, momentum=0.1, eps=1e-5)
    yr.backward(dy.double())
    # device: a bf16 module
    bn = torch.nn.BatchNorm2d(C, momentum=0.1, eps=1e-5, track_running_stats=track).bfloat16()
    with torch.no_grad():
        bn.weight.copy_(w)
        bn.bias.copy_(b)
        if track:
            bn.running_mean.copy_(rm0)
            bn.running_var.copy_(rv0)
    bn = bn.to(X).train()
    xd = x.to(X).requires_grad_(True)
    xdna_train.reset_mapped_cpu_stats()
    yd = bn(xd)
    yd.backward(dy.to(X))
    torch.xdna.synchronize()
    stats = xdna_train.mapped_cpu_stats()
    assert stats.get("hip_batch_norm_train.fwd.run", {}).get("calls", 0) == 1, stats
    assert stats.get("hip_batch_norm_train.bwd.run", {}).get("calls", 0) == 1, stats
    assert not any(k.startswith("aten::native_batch_norm") for k in stats), stats
    check_bf16(bits(yd), yr.detach().numpy(), what="batch_norm out")
    check_bf16(bits(xd.grad), xr.grad.numpy(), what="batch_norm dx")
    check_param_grads(((bn.weight.grad, wr.grad, "dweight"), (bn.bias.grad, br.grad, "dbias")), torch.bfloat16)
    if track:
        for got, ref, name in ((bn.running_mean, rmr, "running_mean"), (bn.running_var, rvr, "running_var")):
            gv = got.detach().cpu().double().numpy()
            rv = ref.numpy()
            tol = oracle.bf16_ulp(rv) + 1e-7
            assert (np.abs(gv - rv) <= tol).all(), (name, np.abs(gv - rv).max())


def _lane_sum_f32(terms):
    """A 64-lane wave's sum of per-image terms as the kernels form it: lane l adds images
    l, l + 64, ... in order, then the lanes' butterfly (xor 32, 16, ..., 1), in float32."""
    t = np.zeros(64, np.float32)
    for b, v in enumerate(np.asarray(terms, np.float32)):
        t[b % 64] = np.float32(t[b % 64] + v)
    for o in (32, 16, 8, 4, 2, 1):
        t = (t + t[np.arange(64) ^ o]).astype(np.float32)
    return t[0]


@pytest.mark.parametrize("act", [0, 1])
@pytest.mark.parametrize("B,C,L", [(40, 16, 81), (3, 8, 1296), (70, 4, 5), (2, 3, 2048)])
def test_instance_norm_register_planes_match_loop_kernels(hip, act, B, C, L):
    """The instance-norm kernels that hold a plane in registers (planes up to 2048 elements)
    against the batch-norm kernels' loop form on the same planes (batch norm over
    [1, B*C, L], the weight repeated per plane, fp32 parameters): y, the saved statistics
    and dx bit for bit, with the activation's mask applied to dy for the batch-norm side;
    dweight / dbias equal to the batch-norm per-plane terms summed in the kernels' order."""
    from gpu_util import stream
    g = torch.Generator().manual_seed(B * L + act)
    x = (torch.randn(B, C, L, generator=g) * 2 + 0.3).bfloat16().cuda()
    dy = torch.randn(B, C, L, generator=g).bfloat16().cuda()
    w = (torch.rand(C, generator=g) + 0.5).bfloat16().cuda()
    b = (torch.randn(C, generator=g) * 0.1).bfloat16().cuda()
    P = B * C
    y = torch.empty_like(x)
    mean, inv = torch.empty(P, device="cuda"), torch.empty(P, device="cuda")
    assert hip.xdna_instance_norm_act_fwd_bf16(x.data_ptr(), w.data_ptr(), b.data_ptr(), 1, y.data_ptr(),
                                               mean.data_ptr(), inv.data_ptr(), B, C, L, 1e-5, act, 0.0,
                                               stream()) == 0
    dx = torch.empty_like(x)
    dw = torch.empty(C, dtype=torch.bfloat16, device="cuda")
    db = torch.empty(C, dtype=torch.bfloat16, device="cuda")
    assert hip.xdna_instance_norm_act_bwd_bf16(dy.data_ptr(), x.data_ptr(), y.data_ptr(), w.data_ptr(), 1,
                                               mean.data_ptr(), inv.data_ptr(), dx.data_ptr(), dw.data_ptr(),
                                               db.data_ptr(), B, C, L, act, 0.0, stream()) == 0
    # the loop kernels: batch norm over the planes
    wp = w.float().repeat(B).contiguous()
    bp = b.float().repeat(B).contiguous()
    y2 = torch.empty_like(x)
    mean2, inv2 = torch.empty(P, device="cuda"), torch.empty(P, device="cuda")
    assert hip.xdna_batch_norm_fwd_bf16(x.data_ptr(), wp.data_ptr(), bp.data_ptr(), 2, y2.data_ptr(),
                                        mean2.data_ptr(), inv2.data_ptr(), 1, P, L, 1e-5, stream()) == 0
    torch.cuda.synchronize()
    if act:
        y2 = torch.where(y2.float() <= 0, torch.zeros_like(y2), y2)
    dy2 = torch.where(y.float() <= 0, torch.zeros_like(dy), dy) if act else dy
    dx2 = torch.empty_like(x)
    dw2 = torch.empty(P, device="cuda")
    db2 = torch.empty(P, device="cuda")
    assert hip.xdna_batch_norm_bwd_bf16(dy2.data_ptr(), x.data_ptr(), wp.data_ptr(), 2, mean2.data_ptr(),
                                        inv2.data_ptr(), dx2.data_ptr(), dw2.data_ptr(), db2.data_ptr(), 1, P, L,
                                        stream()) == 0
    torch.cuda.synchronize()
    for got, want, name in ((y, y2, "y"), (dx, dx2, "dx")):
        assert torch.equal(got.view(torch.int16), want.contiguous().view(torch.int16)), name
    assert torch.equal(mean, mean2) and torch.equal(inv, inv2), "statistics"
    tw = dw2.view(B, C).cpu().numpy()
    tb = db2.view(B, C).cpu().numpy()
    want_w = torch.tensor([_lane_sum_f32(tw[:, c]) for c in range(C)]).bfloat16()
    want_b = torch.tensor([_lane_sum_f32(tb[:, c]) for c in range(C)]).bfloat16()
    assert torch.equal(dw.cpu().view(torch.int16), want_w.view(torch.int16)), "dweight"
    assert torch.equal(db.cpu().view(torch.int16), want_b.view(torch.int16)), "dbias"
