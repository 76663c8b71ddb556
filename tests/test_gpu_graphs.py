"""Graph capture of xdna work: a captured conv + linear + Adam training step replays with
the results of the same step run eagerly, replay after replay, with eager work and
synchronizations between the replays; the private allocator pool keeps the graph's
memory away from eager allocations."""
import pytest
import torch

import xdna_train  # noqa: F401  (registers the device)

pytestmark = pytest.mark.gpu
X = torch.device("xdna")


def _model(seed):
    torch.manual_seed(seed)
    m = torch.nn.Sequential(torch.nn.Conv2d(64, 64, 3, padding=1), torch.nn.ReLU(),
                            torch.nn.Conv2d(64, 32, 3, padding=1), torch.nn.Flatten(),
                            torch.nn.Linear(32 * 12 * 12, 64)).bfloat16()
    return m


def _step_fn(m, opt, x, t):
    def step():
        opt.zero_grad(set_to_none=True)
        loss = torch.nn.functional.mse_loss(m(x).float(), t)
        loss.backward()
        opt.step()
        return loss
    return step


def test_captured_training_step_matches_eager():
    g = torch.Generator().manual_seed(1)
    x_cpu = torch.randn(8, 64, 12, 12, generator=g).bfloat16()
    t_cpu = torch.randn(8, 64, generator=g)
    # eager reference run
    m_e = _model(0).to(X)
    opt_e = torch.optim.Adam(m_e.parameters(), lr=1e-3, fused=True, capturable=True)
    step_e = _step_fn(m_e, opt_e, x_cpu.to(X), t_cpu.to(X))
    eager_losses = [float(step_e()) for _ in range(6)]
    eager_params = [p.detach().cpu() for p in m_e.parameters()]
    # graphed run: two eager warm-up steps, capture the third, replay the rest
    m_g = _model(0).to(X)
    opt_g = torch.optim.Adam(m_g.parameters(), lr=1e-3, fused=True, capturable=True)
    x, t = x_cpu.to(X), t_cpu.to(X)
    step_g = _step_fn(m_g, opt_g, x, t)
    losses = [float(step_g()) for _ in range(2)]
    graph = torch.xdna.Graph()
    with torch.xdna.graph(graph):
        loss = step_g()
    for i in range(4):
        graph.replay()
        # eager work between the replays, on fresh allocations
        junk = torch.randn(256, 256, device=X).bfloat16()
        _ = (junk @ junk).sum()
        torch.xdna.synchronize()
        losses.append(float(loss))
    print("eager", eager_losses, "graph", losses, flush=True)
    assert losses == eager_losses
    for pe, pg in zip(eager_params, m_g.parameters()):
        assert torch.equal(pe, pg.detach().cpu())
    graph.reset()
    torch.xdna.synchronize()


def _stat_calls(name):
    return xdna_train.mapped_cpu_stats().get(name, {}).get("calls", 0)


def test_captured_step_adopts_trainable_forms():
    """The trainable conv weights' prepared forms made by the eager optimizer step are
    adopted by the capture (no preparation recorded per weight); the captured optimizer
    step prepares them again in one launch; replays match the eager run bit for bit (the
    test above) and the capture records no per-weight preparation."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(8, 64, 12, 12, generator=g).bfloat16().to(X)
    t = torch.randn(8, 64, generator=g).to(X)
    m = _model(0).to(X)
    opt = torch.optim.Adam(m.parameters(), lr=1e-3, fused=True, capturable=True)
    step = _step_fn(m, opt, x, t)
    for _ in range(2):
        step()
    torch.xdna.synchronize()
    prep0 = _stat_calls("hip_conv3x3.weights")
    adopt0 = _stat_calls("hip_conv3x3.weights_graph")
    refresh0 = _stat_calls("hip_conv3x3.weights_graph_step_refresh")
    graph = torch.xdna.Graph()
    with torch.xdna.graph(graph):
        step()
    assert _stat_calls("hip_conv3x3.weights") == prep0, "the capture prepared a weight itself"
    # both forward forms and the second conv's input-gradient form (the first conv's input
    # needs no gradient)
    assert _stat_calls("hip_conv3x3.weights_graph") - adopt0 == 3
    assert _stat_calls("hip_conv3x3.weights_graph_step_refresh") - refresh0 == 1
    graph.reset()
    torch.xdna.synchronize()


@pytest.mark.parametrize("between", ["eager_optimizer", "weight_write"])
def test_replays_see_eager_writes_of_adopted_trainable_weights(between):
    """A graph of forward + backward only (the optimizer steps eagerly between replays),
    or of the whole step with the weights rescaled eagerly between replays: the adopted
    forms are prepared again before each replay that needs it, so every replay computes
    with the weights' current values, bit for bit as the same sequence run eagerly."""
    g = torch.Generator().manual_seed(4)
    x_cpu = torch.randn(8, 64, 12, 12, generator=g).bfloat16()
    t_cpu = torch.randn(8, 64, generator=g)

    def run(graphed):
        m = _model(1).to(X)
        opt = torch.optim.Adam(m.parameters(), lr=1e-3, fused=True, capturable=True)
        x, t = x_cpu.to(X), t_cpu.to(X)

        def fwd_bwd():
            opt.zero_grad(set_to_none=False)
            loss = torch.nn.functional.mse_loss(m(x).float(), t)
            loss.backward()
            return loss

        def full():
            loss = fwd_bwd()
            opt.step()
            return loss

        body = fwd_bwd if between == "eager_optimizer" else full
        losses = []
        for _ in range(2):
            losses.append(float(full()))
        if graphed:
            graph = torch.xdna.Graph()
            with torch.xdna.graph(graph):
                loss = body()
        for _ in range(4):
            if graphed:
                graph.replay()
            else:
                loss = body()
            if between == "eager_optimizer":
                opt.step()
            else:
                with torch.no_grad():
                    m[0].weight.mul_(0.75)
                    m[2].weight.mul_(1.25)
            torch.xdna.synchronize()
            losses.append(float(loss))
        params = [p.detach().cpu() for p in m.parameters()]
        if graphed:
            graph.reset()
            torch.xdna.synchronize()
        return losses, params

    le, pe = run(False)
    lg, pg = run(True)
    print(between, "eager", le, "graph", lg, flush=True)
    assert lg == le
    for a, b in zip(pe, pg):
        assert torch.equal(a, b)


def _replayed_params(overlap):
    """Two eager steps, a captured third, three replays; the weight gradients of the
    3x3 layers whose input gradient is also needed run beside it when `overlap`."""
    nat = xdna_train.device.native()
    before = nat.wgrad_overlap()
    nat.set_wgrad_overlap(overlap)
    try:
        g = torch.Generator().manual_seed(5)
        x, t = torch.randn(8, 64, 12, 12, generator=g).bfloat16().to(X), torch.randn(8, 64, generator=g).to(X)
        m = _model(3).to(X)
        opt = torch.optim.Adam(m.parameters(), lr=1e-3, fused=True, capturable=True)
        step = _step_fn(m, opt, x, t)
        for _ in range(2):
            step()
        xdna_train.reset_mapped_cpu_stats()
        graph = torch.xdna.Graph()
        with torch.xdna.graph(graph):
            loss = step()
        beside = _stat_calls("hip_conv3x3.dw_rows.beside_dx")
        losses = []
        for _ in range(3):
            graph.replay()
            torch.xdna.synchronize()
            losses.append(float(loss))
        return beside, losses, [p.detach().cpu() for p in m.parameters()]
    finally:
        nat.set_wgrad_overlap(before)


def test_captured_weight_gradient_beside_input_gradient():
    """With the opt-in overlap, the second conv's weight gradient in a captured step forks
    onto the side stream (its input gradient is needed too) and joins before the
    optimizer: the replays give the bits of the same step captured on one stream."""
    print("graph: weight gradient beside the input gradient", flush=True)
    beside, losses, params = _replayed_params(1)
    beside0, losses0, params0 = _replayed_params(0)
    assert beside == 1 and beside0 == 0
    assert losses == losses0
    for a, b in zip(params, params0):
        assert torch.equal(a, b)
