"""Caches of prepared conv weights and kept packs follow every write, and never hand a
captured graph a buffer it does not own.

Ports of the reference's weight-cache checks (tests/run_conv3x3w_torch.py:60-157): every
in-place update path of a weight, `.data` writes (which leave the version counter alone
and are seen only through the per-allocation write epoch,
torch_xdna_device.cpp:493, 576, 620-633, 2222), optimizer steps, and a frozen weight
prepared once.  "Uncached" results come from the same call after the caches are emptied.
Plus: graph capture with a frozen conv across empty_cache and weight updates between
replays, the tensor-lr fused Adam under capture, out= products written in place, and the
host wait deadline.
"""
import ctypes

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

import xdna_train
from xdna_train import hip_abi

pytestmark = pytest.mark.gpu
X = torch.device("xdna")


@pytest.fixture(scope="module", autouse=True)
def xdna():
    assert xdna_train.is_available(), "xdna device not available on the GPU box"
    xdna_train.set_npu_mode(2)
    return xdna_train


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16)


def _same(a, b):
    return all(torch.equal(_bits(u), _bits(v)) for u, v in zip(a, b))


def _counts():
    st = xdna_train.mapped_cpu_stats()
    return (st.get("hip_conv3x3.weights", {}).get("calls", 0),
            st.get("hip_conv3x3.weights_hit", {}).get("calls", 0))


def _data():
    g = torch.Generator().manual_seed(1)
    x = torch.randn(4, 64, 12, 12, generator=g).bfloat16().to(X)
    dy = torch.randn(4, 64, 12, 12, generator=g).bfloat16().to(X)
    return x, dy


def _fwd_dx(conv, x, dy):
    xx = x.clone().requires_grad_()
    if conv.weight.grad is not None:
        conv.weight.grad = None
    y = conv(xx)
    y.backward(dy)
    out = [y.detach().clone(), xx.grad.clone()]
    if conv.weight.requires_grad:
        out.append(conv.weight.grad.clone())
    return out


def _uncached(conv, x, dy):
    torch.xdna.empty_cache()
    return _fwd_dx(conv, x, dy)


UPDATES = [
    ("add_", lambda w, o: w.add_(0.05)),
    ("mul_", lambda w, o: w.mul_(1.5)),
    ("copy_", lambda w, o: w.copy_(o)),
    ("addcmul_", lambda w, o: w.addcmul_(o, o, value=0.1)),
    ("fill_", lambda w, o: w.fill_(0.03)),
    ("data.add_", lambda w, o: w.data.add_(0.05)),
    ("data.copy_", lambda w, o: w.data.copy_(o)),
    ("data.mul_", lambda w, o: w.data.mul_(-0.5)),
]


@pytest.mark.parametrize("frozen", [True, False], ids=["frozen", "trainable"])
@pytest.mark.parametrize("name,update", UPDATES, ids=[u[0] for u in UPDATES])
def test_weight_updates_are_seen(name, update, frozen):
    torch.manual_seed(0)
    x, dy = _data()
    conv = nn.Conv2d(64, 64, 3, padding=1, bias=False).bfloat16().to(X)
    conv.weight.requires_grad_(not frozen)
    other = torch.randn(conv.weight.shape).bfloat16().to(X)
    _fwd_dx(conv, x, dy)  # warm: the frozen forms are cached now
    before = _fwd_dx(conv, x, dy)
    v0 = conv.weight._version
    with torch.no_grad():
        update(conv.weight, other)
    got = _fwd_dx(conv, x, dy)
    ref = _uncached(conv, x, dy)
    assert _same(got, ref), f"{name}: cached result differs from the uncached one"
    # the update changed the output (a stale cache entry would have kept it)
    assert not torch.equal(_bits(before[0]), _bits(got[0]))
    if name.startswith("data."):
        # the version counter does not see a .data write; the write epoch does
        assert conv.weight._version == v0


def test_frozen_weight_prepared_once_then_hit():
    torch.manual_seed(0)
    x, dy = _data()
    conv = nn.Conv2d(64, 64, 3, padding=1, bias=False).bfloat16().to(X)
    conv.weight.requires_grad_(False)
    torch.xdna.empty_cache()
    xdna_train.reset_mapped_cpu_stats()
    xx = x.clone().requires_grad_()
    for _ in range(5):
        conv(xx).backward(dy)
    prep, hit = _counts()
    assert (prep, hit) == (2, 8), (prep, hit)  # forward and input-gradient forms once each


def test_trainable_weight_prepared_once_per_optimizer_step():
    """Trainable weights are prepared once (both forms, one launch) until a write: steps
    without an optimizer update hit the cache.  A fused optimizer step makes both forms
    again itself (one launch for all the conv weights it wrote) and the next forward and
    input gradient find them; with that refresh off (XDNA_ADAM_PREP=0) the update's epoch
    bump makes the next forward prepare them."""
    torch.manual_seed(0)
    x, dy = _data()
    conv = nn.Conv2d(64, 64, 3, padding=1, bias=False).bfloat16().to(X)
    opt = torch.optim.Adam(conv.parameters(), lr=0.05)
    torch.xdna.empty_cache()
    xdna_train.reset_mapped_cpu_stats()
    for _ in range(3):
        conv(x).backward(dy)
    st = {k: v["calls"] for k, v in xdna_train.mapped_cpu_stats().items()}
    # x needs no gradient: one forward lookup per step (one preparation, then hits)
    assert _counts() == (1, 2), st
    xdna_train.reset_mapped_cpu_stats()
    opt.step()
    st = {k: v["calls"] for k, v in xdna_train.mapped_cpu_stats().items()}
    assert st.get("hip_conv3x3.weights_refresh", 0) == 1, st
    # a write outside the optimizer after the refresh: the next forward prepares again
    with torch.no_grad():
        conv.weight.data.mul_(0.5)
    xdna_train.reset_mapped_cpu_stats()
    got = _fwd_dx(conv, x, dy)
    assert _counts() == (1, 1), xdna_train.mapped_cpu_stats()
    assert _same(got, _uncached(conv, x, dy))
    # the refreshed forms serve the next forward and input gradient
    conv(x).backward(dy)
    opt.step()
    xdna_train.reset_mapped_cpu_stats()
    got = _fwd_dx(conv, x, dy)
    st = {k: v["calls"] for k, v in xdna_train.mapped_cpu_stats().items()}
    assert _counts() == (0, 2), st
    assert _same(got, _uncached(conv, x, dy))


def test_eager_after_graph_replay_uses_the_replayed_weights():
    """A replayed optimizer step writes the weights with no host code: the eager forms
    cached before the capture must not be served after a replay."""
    torch.manual_seed(0)
    x, dy = _data()
    conv = nn.Conv2d(64, 64, 3, padding=1, bias=False).bfloat16().to(X)
    opt = torch.optim.Adam(conv.parameters(), lr=0.05, fused=True, capturable=True)

    def step():
        opt.zero_grad(set_to_none=True)
        conv(x).backward(dy)
        opt.step()

    step()
    step()  # eager: the forms of the current weights are cached
    graph = torch.xdna.Graph()
    with torch.xdna.graph(graph):
        step()
    for _ in range(3):
        graph.replay()
    torch.xdna.synchronize()
    got = _fwd_dx(conv, x, dy)
    assert _same(got, _uncached(conv, x, dy))
    graph.reset()


@pytest.mark.parametrize("frozen", [True, False], ids=["frozen", "trainable"])
def test_views_of_one_storage_are_different_weights(frozen):
    """w and w.transpose(2, 3) share storage, offset, shape, version counter and write
    epoch; only their strides differ.  Each conv must compute with its own view's values
    (forward and input gradient against the float64 oracle), in either call order."""
    import oracle
    from gpu_util import check_bf16
    g = torch.Generator().manual_seed(5)
    w_cpu = (torch.randn(64, 64, 3, 3, generator=g) * 0.05).bfloat16()
    w = w_cpu.to(X).requires_grad_(not frozen)
    x, dy = _data()
    xb = x.cpu().view(torch.int16).numpy().view(np.uint16)
    dyb = dy.cpu().view(torch.int16).numpy().view(np.uint16)
    for label, view in (("w", w), ("w.T", w.transpose(2, 3)), ("w again", w), ("w.T again", w.transpose(2, 3))):
        xx = x.clone().requires_grad_()
        y = F.conv2d(xx, view, None, 1, 1)
        y.backward(dy)
        vb = view.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
        check_bf16(_bits(y).numpy().view(np.uint16), oracle.conv3x3_fwd(xb, vb), what=f"{label} forward")
        check_bf16(_bits(xx.grad).numpy().view(np.uint16), oracle.conv3x3_dgrad(dyb, vb), what=f"{label} dgrad")


def test_released_graph_drops_its_cache_entries():
    """Releasing a captured graph drops the prepared weights and kept packs made under its
    capture tag; the eager entries stay."""
    torch.manual_seed(0)
    x, dy = _data()
    frozen = nn.Conv2d(64, 64, 3, padding=1).bfloat16().to(X).requires_grad_(False)
    conv = nn.Conv2d(64, 64, 3, padding=1).bfloat16().to(X)
    C = xdna_train.device.native()

    def step():
        xx = x.clone().requires_grad_()
        conv(frozen(xx)).backward(dy)

    step()
    eager = C.cache_stats(0)
    graph = torch.xdna.Graph()
    with torch.xdna.graph(graph):
        step()
    graph.replay()
    torch.xdna.synchronize()
    assert C.cache_stats(graph.pool)[0] > 0  # trainable forms prepared inside the capture
    pool = graph.pool
    graph.reset()
    torch.xdna.synchronize()
    assert C.cache_stats(pool) == [0, 0, 0, 0]
    assert C.cache_stats(0)[0] >= 1 and eager[0] >= 1


@pytest.mark.parametrize("make", [
    lambda p: torch.optim.SGD(p, lr=0.5),
    lambda p: torch.optim.SGD(p, lr=0.5, momentum=0.9, weight_decay=0.1),
    lambda p: torch.optim.Adam(p, lr=0.05),
    lambda p: torch.optim.AdamW(p, lr=0.05),
], ids=["sgd", "sgd_mom_wd", "adam", "adamw"])
def test_optimizer_steps_are_seen(make):
    torch.manual_seed(0)
    x, dy = _data()
    conv = nn.Conv2d(64, 64, 3, padding=1, bias=False).bfloat16().to(X)
    opt = make(conv.parameters())
    prev = None
    for _ in range(4):
        got = _fwd_dx(conv, x, dy)
        ref = _uncached(conv, x, dy)
        assert _same(got, ref)
        assert prev is None or not torch.equal(_bits(prev), _bits(got[0]))
        prev = got[0]
        opt.zero_grad()
        conv(x).backward(dy)
        opt.step()


def _graph_model(seed):
    torch.manual_seed(seed)
    m = nn.Sequential(nn.Conv2d(32, 64, 3, padding=1), nn.ReLU(),
                      nn.Conv2d(64, 64, 3, padding=1), nn.ReLU(),
                      nn.Conv2d(64, 32, 3, padding=1)).bfloat16()
    # frozen middle layer: both its forms go through the weight cache eagerly, and its
    # input gradient is needed by the first layer
    m[2].weight.requires_grad_(False)
    m[2].bias.requires_grad_(False)
    return m.to(X)


def test_capture_with_frozen_conv_survives_empty_cache_and_sees_updates():
    """A capture adopts the eager prepared form of a frozen weight instead of recording a
    preparation (the graph keeps it alive): empty_cache between replays cannot free it,
    and a write to the frozen weight between replays makes the next replay prepare it again
    first, so every replay matches the eager run exactly."""
    g = torch.Generator().manual_seed(3)
    x_cpu = torch.randn(8, 32, 12, 12, generator=g).bfloat16()
    t_cpu = torch.randn(8, 32, 12, 12, generator=g)
    w_new = torch.randn(64, 64, 3, 3, generator=g).bfloat16() * 0.05
    n_steps, update_after = 7, 4

    def run(graphed):
        m = _graph_model(0)
        opt = torch.optim.Adam([p for p in m.parameters() if p.requires_grad], lr=1e-3,
                               fused=True, capturable=True)
        x, t = x_cpu.to(X), t_cpu.to(X)

        def step():
            opt.zero_grad(set_to_none=True)
            loss = F.mse_loss(m(x).float(), t)
            loss.backward()
            opt.step()
            return loss

        losses = []
        if not graphed:
            for i in range(n_steps):
                losses.append(float(step()))
                if i == update_after:
                    m[2].weight.data.copy_(w_new.to(X))
            return losses, [p.detach().cpu() for p in m.parameters()]
        for _ in range(2):
            losses.append(float(step()))
        graph = torch.xdna.Graph()
        xdna_train.reset_mapped_cpu_stats()
        with torch.xdna.graph(graph):
            loss = step()
        st = xdna_train.mapped_cpu_stats()
        assert st.get("hip_conv3x3.weights_graph", {}).get("calls", 0) >= 1, st
        for i in range(2, n_steps):
            torch.xdna.empty_cache()  # frees every cached block the eager warm-up left
            junk = [torch.randn(64, 64, 3, 3, device=X).bfloat16() for _ in range(8)]
            graph.replay()
            del junk
            torch.xdna.synchronize()
            losses.append(float(loss))
            if i == 2:
                # the first replay prepares the adopted trainable forms again (the captured
                # optimizer step moved their version counters); from here on only the
                # frozen weight's update asks for a refresh
                xdna_train.reset_mapped_cpu_stats()
            if i == update_after:
                m[2].weight.data.copy_(w_new.to(X))
        out = [p.detach().cpu() for p in m.parameters()]
        st = xdna_train.mapped_cpu_stats()
        assert st.get("hip_conv3x3.weights_graph_refresh", {}).get("calls", 0) == 1, st
        graph.reset()
        return losses, out

    eager_losses, eager_params = run(False)
    graph_losses, graph_params = run(True)
    print("eager", eager_losses, "graph", graph_losses, flush=True)
    assert graph_losses == eager_losses
    assert _same(eager_params, graph_params)
    torch.xdna.synchronize()


def test_tensor_lr_adam_matches_cpu_and_captures():
    """The tensor-lr overload reads lr on the device (no host read): bit-exact with torch's
    CPU fused Adam given the same tensor lr, and capturable."""
    torch.manual_seed(0)
    p_cpu = torch.randn(4099).bfloat16()
    grads = [torch.randn(4099).bfloat16() for _ in range(3)]
    ref = p_cpu.clone().requires_grad_()
    opt_c = torch.optim.Adam([ref], lr=torch.tensor(2e-3), fused=True)
    for gr in grads:
        ref.grad = gr.clone()
        opt_c.step()
    p = p_cpu.clone().to(X).requires_grad_()
    opt = torch.optim.Adam([p], lr=torch.tensor(2e-3, device=X), fused=True, capturable=True)
    xdna_train.reset_mapped_cpu_stats()
    p.grad = grads[0].to(X)
    opt.step()
    assert xdna_train.mapped_cpu_stats().get("hip_adam.run", {}).get("calls", 0) == 1
    static_grad = p.grad
    graph = torch.xdna.Graph()
    with torch.xdna.graph(graph):
        opt.step()
    for gr in grads[1:]:
        static_grad.copy_(gr.to(X))
        graph.replay()
    torch.xdna.synchronize()
    assert torch.equal(_bits(p), _bits(ref))
    graph.reset()


def test_out_variants_write_in_place():
    torch.manual_seed(0)
    a = torch.randn(300, 200).bfloat16().to(X)
    b = torch.randn(200, 170).bfloat16().to(X)
    c = torch.randn(170).bfloat16().to(X)
    xdna_train.reset_mapped_cpu_stats()
    out = torch.empty(300, 170, dtype=torch.bfloat16, device=X)
    ptr = out.data_ptr()
    torch.mm(a, b, out=out)
    assert out.data_ptr() == ptr and torch.equal(_bits(out), _bits(torch.mm(a, b)))
    out2 = torch.empty(300, 170, dtype=torch.bfloat16, device=X)
    torch.addmm(c, a, b, beta=0.5, alpha=2.0, out=out2)
    assert torch.equal(_bits(out2), _bits(torch.addmm(c, a, b, beta=0.5, alpha=2.0)))
    ba = torch.randn(3, 40, 50).bfloat16().to(X)
    bb = torch.randn(3, 50, 60).bfloat16().to(X)
    out3 = torch.empty(0, dtype=torch.bfloat16, device=X)
    torch.bmm(ba, bb, out=out3)
    assert out3.shape == (3, 40, 60) and torch.equal(_bits(out3), _bits(torch.bmm(ba, bb)))
    st = xdna_train.mapped_cpu_stats()
    for k in ("hip_gemm.mm_out.run", "hip_gemm.addmm_out.run", "hip_gemm.bmm_out.run"):
        assert st.get(k, {}).get("calls", 0) == 1, (k, st)
    # out = self (the bias) takes the copy path and still computes beta*self + alpha*a.b
    s = torch.randn(300, 170).bfloat16().to(X)
    expect = torch.addmm(s, a, b)
    torch.addmm(s, a, b, out=s)
    assert torch.equal(_bits(s), _bits(expect))
    # a transposed out view is written through its strides
    outt = torch.empty(170, 300, dtype=torch.bfloat16, device=X).t()
    torch.mm(a, b, out=outt)
    assert torch.equal(_bits(outt), _bits(torch.mm(a, b)))


def test_wait_deadline_times_out_on_long_work_then_recovers(hip, stream):
    """A 1 ms deadline on a stream that has several milliseconds of queued GEMMs: the wait
    reports a timeout (-2, not an error), poisons the process, and after the queued work
    drains (it always completes) the state is reset.  Forced from the host: the kernels
    are ordinary, bounded launches."""
    n = 8192
    a = torch.randn(n, n, device="cuda").bfloat16()
    b = torch.randn(n, n, device="cuda").bfloat16()
    c = torch.empty(n, n, device="cuda", dtype=torch.bfloat16)
    torch.cuda.synchronize()
    old = hip.xdna_hip_wait_timeout_ms()
    hip.xdna_hip_reset_failure_state()
    try:
        for _ in range(4):  # ~1.1 TFLOP each
            rc = hip.xdna_gemm_bf16(a.data_ptr(), b.data_ptr(), c.data_ptr(), None, 1, n, n, n, n, 1, 0, n,
                                    1, 0, n, 1, 0, 0, 0, 0, 1.0, 0.0, stream)
            assert rc == 0, hip_abi.last_error()
        assert hip.xdna_hip_set_wait_timeout_ms(1) == 0
        rc = hip.xdna_hip_stream_synchronize(ctypes.c_void_p(stream))
        msg = hip_abi.last_error()
        print("deadline wait:", rc, msg, flush=True)
        assert rc == -2 and msg.startswith("deadline:") and hip.xdna_hip_poisoned() == 1
    finally:
        torch.cuda.synchronize()  # the queued GEMMs finish on their own
        hip.xdna_hip_set_wait_timeout_ms(old)
        hip.xdna_hip_reset_failure_state()
    assert hip.xdna_hip_stream_synchronize(ctypes.c_void_p(stream)) == 0
    assert hip.xdna_hip_max_wait_ms() >= 0.0
