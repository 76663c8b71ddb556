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
