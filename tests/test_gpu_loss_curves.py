"""Training on xdna follows the reference's CPU bf16 path: 200-step loss curves of BASELINE
configs 1, 3, 4 and 5 against the same seeded run on torch.device("cpu") in bf16 (configs
3 and 5 against CPU runs recorded once by tests/golden/make_loss_curves.py, whose five
200-step CPU runs exceed a test's time; configs 1 and 4 run their CPU runs here), plus
config 4's first-step gradients against an fp32 computation.

Curves are compared as the reference compares them (benchmarks/loss_curve_compare.py:
25-36): means over windows of max(10, steps/10) steps.  The CPU run uses Adam's fused
kernel, which is what the reference executes for an xdna model (its pre-hook picks
fused=True and the CPU kernel runs it, device.py:408-436); the xdna run leaves the choice
to the backend's pre-hook.  The bar:

* config 1, config 3's first two windows and the first window of configs 4 and 5: within
  1 % of the CPU run (north_star's bar), with an absolute floor of 1e-4 x the first window
  for losses that have collapsed to rounding level (config 1 trains to ~0);
* every window of every config: within 1 %, or within 1.5x the CPU's own rounding spread
  up to that window: the largest deviation, over the windows so far, of three CPU runs
  whose only difference is one weight moved by one bf16 ulp (a trajectory that rounding
  has moved stays moved, so the envelope is cumulative).  This is the reference's
  criterion ("stays within the run-to-run spread", loss_curve_compare.py:10-14).  On
  config 4 that spread is ~3 % (measured), on config 3 past step 40 up to ~27 %: rounding
  alone moves those curves by more than 1 %, so no implementation that is not
  bit-identical to the CPU's kernels can meet a flat 1 % there.

The CPU's default single-tensor Adam (the reference's plain CPU path) is run too, and the
xdna curve must be as close to it as the CPU's fused run is, within 1 % more.  Path
counters prove the HIP kernels ran (tests/quick_check.py:34-84); every curve descends.
"""
import json
import statistics
from pathlib import Path

import pytest
import torch

import bench
import xdna_train

pytestmark = pytest.mark.gpu
X = torch.device("xdna")
CPU = torch.device("cpu")


@pytest.fixture(scope="module", autouse=True)
def xdna():
    assert xdna_train.is_available(), "xdna device not available on the GPU box"
    xdna_train.set_npu_mode(2)
    return xdna_train


def _nudge(model, where):
    """Moves one element of the first trainable weight by one bf16 ulp."""
    p = next(q for q in model.parameters() if q.requires_grad and q.numel() > 1)
    flat = p.data.view(-1)
    i = [0, flat.numel() // 2, flat.numel() - 1][where]
    with torch.no_grad():
        v = flat[i:i + 1].float()
        flat[i:i + 1] = (v * (1 + 2.0 ** -7)).bfloat16()


def _curve(build, device, steps, fused, nudge=None):
    step, model = build(torch, device, fused=fused)
    if nudge is not None:
        _nudge(model, nudge)
    return [float(step().detach()) for _ in range(steps)]


def _windows(losses):
    w = max(10, len(losses) // 10)
    return [statistics.mean(losses[lo:lo + w]) for lo in range(0, len(losses) - w + 1, w)]


def _check(name, build, steps, counters, strict_windows, fixture=None):
    """fixture: the CPU runs precomputed by tests/golden/make_loss_curves.py (fused Adam,
    default Adam, three 1-ulp spread runs), instead of running them here."""
    xdna_train.reset_mapped_cpu_stats()
    dev = _curve(build, X, steps, None)
    st = xdna_train.mapped_cpu_stats()
    for k in counters:
        assert st.get(k, {}).get("calls", 0) >= steps, (k, st.get(k))
    if fixture is not None:
        cpu, spread_runs, cpu_default = fixture["cpu_fused"], fixture["spread"], fixture["cpu_default"]
        assert fixture["steps"] == steps and len(cpu) == steps
    else:
        cpu = _curve(build, CPU, steps, True)
        spread_runs = [_curve(build, CPU, steps, True, nudge=w) for w in (0, 1, 2)]
        cpu_default = _curve(build, CPU, steps, None)
    assert dev[-1] < dev[0] and cpu[-1] < cpu[0], "the loss did not descend"

    wd, wc, wcd = _windows(dev), _windows(cpu), _windows(cpu_default)
    spread = [max(abs(_windows(r)[i] - wc[i]) for r in spread_runs) for i in range(len(wc))]
    floor = 1e-4 * abs(wc[0])
    rel = [abs(a - b) / max(abs(b), floor) for a, b in zip(wd, wc)]
    rel_spread = [s / max(abs(b), floor) for s, b in zip(spread, wc)]
    rel_spread = [max(rel_spread[:i + 1]) for i in range(len(rel_spread))]  # running envelope
    print(f"{name}: xdna windows     {[f'{v:.6g}' for v in wd]}", flush=True)
    print(f"{name}: cpu windows      {[f'{v:.6g}' for v in wc]}", flush=True)
    print(f"{name}: rel diff         {[f'{v:.2e}' for v in rel]}", flush=True)
    print(f"{name}: cpu 1-ulp spread {[f'{v:.2e}' for v in rel_spread]}", flush=True)
    for i in range(strict_windows if strict_windows is not None else len(wc)):
        assert rel[i] <= 0.01, f"{name}: window {i} differs from the CPU by {rel[i]:.2%} (> 1 %)"
    for i, (r, s) in enumerate(zip(rel, rel_spread)):
        assert r <= max(0.01, 1.5 * s), \
            f"{name}: window {i} differs by {r:.2%}, beyond 1 % and 1.5x the CPU's 1-ulp spread ({s:.2%})"
    # against the CPU's default (single-tensor) Adam: no further off than the CPU's fused run
    rel_d = [abs(a - b) / max(abs(b), floor) for a, b in zip(wd, wcd)]
    rel_fd = [abs(a - b) / max(abs(b), floor) for a, b in zip(wc, wcd)]
    print(f"{name}: vs cpu default Adam {[f'{v:.2e}' for v in rel_d]} (cpu fused vs default "
          f"{[f'{v:.2e}' for v in rel_fd]})", flush=True)
    for i, (r, f) in enumerate(zip(rel_d, rel_fd)):
        assert r <= 0.01 + 1.5 * max(f, rel_spread[i]), f"{name}: window {i} vs CPU default Adam {r:.2%}"


@pytest.mark.timeout(300)
def test_c1_conv_200_steps():
    _check("C1", bench.build_c1, 200, ("hip_conv3x3.fwd.run", "hip_conv3x3.dw_rows.run", "hip_adam.run"),
           strict_windows=None)


@pytest.mark.timeout(400)
def test_c4_style_200_steps():
    _check("C4", bench.build_style, 200,
           ("hip_conv3x3.fwd.run", "hip_conv3x3.dx.run", "hip_conv3x3.dw_rows.run", "hip_gemm.bmm.run",
            "hip_adam.run"), strict_windows=1)


@pytest.mark.timeout(400)
def test_c4_style_with_fused_loss_region_200_steps():
    """Config 4 with its loss through xdna_train.regions.frozen_feature_loss on xdna; on the
    CPU the region declines and the same loss runs as eager ops, so the reference curve is
    the plain CPU bf16 run."""
    build = lambda torch, device, fused: bench.build_style(torch, device, fused=fused, region=True)
    _check("C4 region", build, 200,
           ("hip_region.conv_relu.run", "hip_region.gram_sqdiff.run", "hip_region.gram_grad.run",
            "hip_region.backward.run", "hip_conv3x3.dw_rows.run", "hip_adam.run"), strict_windows=1)


def _fixture(name):
    path = Path(__file__).resolve().parent / "golden" / "loss_curves.json"
    data = json.loads(path.read_text())
    print(f"{name}: CPU curves from {path.name} (torch {data['meta']['torch']}, {data['meta']['threads']} threads, "
          f"{data['meta']['cpu']})", flush=True)
    return data[name.lower()]


@pytest.mark.timeout(300)
def test_c3_mlp_200_steps():
    """BASELINE config 3 (MLP, x [8192,1024], MSE, Adam): 200 steps against the CPU bf16
    runs recorded by tests/golden/make_loss_curves.py (five 200-step CPU runs do not fit the
    test's time).  The first 40 steps (two windows) within a flat 1 %; from step 40 on the
    run is chaotic (the loss oscillates, and the CPU's own run with one weight moved by one
    ulp leaves it by 1.7 % in steps 40-59 and by over 20 % later), so later windows take
    the spread criterion, as config 4's do."""
    _check("C3", bench.build_mlp, 200, ("hip_gemm.addmm.run", "hip_gemm.mm.run", "hip_adam.run"),
           strict_windows=2, fixture=_fixture("C3"))


@pytest.mark.timeout(300)
def test_c5_resnet18_200_steps():
    """BASELINE config 5 (ResNet-18, B128 3x64x64, CE, Adam): 200 steps against the recorded
    CPU bf16 runs.  Every conv direction, the training batch norms and the Adam step run on
    the HIP kernels."""
    _check("C5", bench.build_resnet, 200,
           ("hip_conv3x3.fwd.run", "hip_conv3x3.dx.run", "hip_conv3x3.dw_rows.run", "hip_conv3x3_s2.fwd.run",
            "hip_conv1x1.fwd.run", "hip_batch_norm_train.fwd.run", "hip_batch_norm_train.bwd.run",
            "hip_adam.run"), strict_windows=1, fixture=_fixture("C5"))


def _style_grads(device, dtype):
    nn = torch.nn
    Generator, VGG = bench.style_models(torch, nn)
    torch.manual_seed(0)
    gen, vgg = Generator().bfloat16(), VGG().bfloat16()
    content = torch.rand(40, 3, 36, 36, generator=torch.Generator().manual_seed(1)).bfloat16()
    style = torch.rand(1, 3, 36, 36, generator=torch.Generator().manual_seed(2)).bfloat16()
    gen, vgg = gen.to(device, dtype), vgg.to(device, dtype)
    for p in vgg.parameters():
        p.requires_grad_(False)
    content, style = content.to(device, dtype), style.to(device, dtype)
    with torch.no_grad():
        grams = {k: bench.gram(v) for k, v in vgg(style, bench.STYLE_TAPS).items()}
        target = vgg(content, (bench.CONTENT_TAP,))[bench.CONTENT_TAP]
    feats = vgg(gen(content), bench.STYLE_TAPS + (bench.CONTENT_TAP,))
    loss = torch.nn.functional.mse_loss(feats[bench.CONTENT_TAP].float(), target.float())
    for k in bench.STYLE_TAPS:
        g = bench.gram(feats[k])
        loss = loss + 1e5 * torch.nn.functional.mse_loss(g, grams[k].expand_as(g))
    loss.backward()
    return [(n, p.grad.detach().double().cpu()) for n, p in gen.named_parameters()]


@pytest.mark.timeout(300)
def test_c4_first_step_gradients_as_accurate_as_cpu_bf16():
    """Both bf16 paths against the same step in fp32 (same bf16 weights and inputs): per
    generator parameter, xdna's relative L2 error is at most 1.25x the CPU bf16 path's plus
    one bf16 rounding (2^-8).  Parameters whose true gradient is zero up to rounding (conv
    biases ahead of an instance norm, |g| < 1e-6 max |g|) carry no signal and are
    skipped."""
    truth = _style_grads(CPU, torch.float32)
    cpu = _style_grads(CPU, torch.bfloat16)
    dev = _style_grads(X, torch.bfloat16)
    gmax = max(float(t.norm()) for _, t in truth)
    checked = 0
    for (name, t), (_, c), (_, d) in zip(truth, cpu, dev):
        nt = float(t.norm())
        if nt < 1e-6 * gmax:
            continue
        ec, ed = float((c - t).norm()) / nt, float((d - t).norm()) / nt
        print(f"{name:26s} cpu-bf16 {ec:.3e} xdna {ed:.3e}", flush=True)
        assert ed <= 1.25 * ec + 2.0 ** -8, f"{name}: xdna gradient error {ed:.3e} vs CPU bf16 {ec:.3e}"
        checked += 1
    assert checked >= 40
