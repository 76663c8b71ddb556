#!/usr/bin/env python3
"""Benchmark of the MI355X xdna hot path on BASELINE.json's workloads.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--skip-cpu] [--skip-style]

Headline (`value`): BASELINE config 2, the 3x3 conv sweep (stride 1, pad 1, bias, bf16;
N {16,40,64} x C_in = C_out {64,128,256,512} x H = W {18,36,72}, 36 shapes).  One step =
forward, dgrad and wgrad (+ bias grad) of every shape through the xdna backend's
convolution ops (the reference's aten::convolution_overrideable /
convolution_backward_overrideable surface).  value = algorithmic fwd+dgrad+wgrad FLOP of
the step (2*N*H*W*C*C*9 per direction, real MACs only) / step time, in TFLOP/s.

Also reported, from the same run:
* "style_net": BASELINE config 4 (Johnson generator + frozen random VGG19 through
  relu4_1, content + Gram style loss, B40 36x36, Adam) in it/s, beside the same step on
  the host CPU in bf16 (the reference's CPU BF16 path: stock PyTorch CPU kernels);
* "adam": fused Adam over config 3's 25,175,040 bf16 parameters (14 B/param), GB/s;
* "mlp": config 3's training step (Linear 1024->4096->4096->1024 with GELU, x [8192,1024],
  MSE, Adam): ms/step and its 1168.2 GFLOP of GEMM per step as TFLOP/s;
* "kernels": per-kernel launches / time / achieved rate from HIP events recorded on the
  launch stream around every hot-kernel launch, over a second pass of the same K steps
  (the event records add GPU time between launches, so `value` is timed without them);
* "roofline": the dominant kernel of the timed region against the MI355X dense bf16
  MFMA peak (2.5 PFLOP/s), or HBM (8 TB/s) for byte-bound kernels;
* "cpu_baseline": PyTorch CPU bf16 conv fwd+dgrad+wgrad (the reference's CPU path) on a
  bounded sample of the sweep, TFLOP/s.

Synthetic data: model seed 0, data seed 1, style image seed 2, sweep shape i seed 1000+i.
One GPU: --gpus above 1 exits.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "pytorch-xdna2_amd"))

METRIC = "it/s style-net b40@36x36; 3x3-conv fwd+dgrad+wgrad BF16 TFLOP/s"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
SWEEP = [(n, c, h) for n in (16, 40, 64) for c in (64, 128, 256, 512) for h in (18, 36, 72)]
ADAM_PARAMS = 25_175_040    # BASELINE config 3 (Linear 1024->4096->4096->1024)


# ---------------------------------------------------------------------------------------
# style-transfer step
# ---------------------------------------------------------------------------------------
def style_models(torch, nn):
    class ConvIN(nn.Sequential):
        def __init__(self, cin, cout, k, stride=1, relu=True):
            layers = [nn.Conv2d(cin, cout, k, stride=stride, padding=k // 2),
                      nn.InstanceNorm2d(cout, affine=True)]
            if relu:
                layers.append(nn.ReLU())
            super().__init__(*layers)

    class Residual(nn.Module):
        def __init__(self, c):
            super().__init__()
            self.body = nn.Sequential(ConvIN(c, c, 3), ConvIN(c, c, 3, relu=False))

        def forward(self, x):
            return x + self.body(x)

    class UpConv(nn.Sequential):
        def __init__(self, cin, cout):
            super().__init__(nn.Upsample(scale_factor=2, mode="nearest"), ConvIN(cin, cout, 3))

    class Generator(nn.Sequential):
        """9x9 3->32, 3x3 s2 32->64, 3x3 s2 64->128, 5 residual blocks, 2 x (nearest x2 +
        3x3 conv) to 64, 32, 9x9 32->3."""

        def __init__(self):
            super().__init__(ConvIN(3, 32, 9), ConvIN(32, 64, 3, 2), ConvIN(64, 128, 3, 2),
                             *[Residual(128) for _ in range(5)], UpConv(128, 64), UpConv(64, 32),
                             nn.Conv2d(32, 3, 9, padding=4))

    # VGG19 conv stack through relu4_1 (random init, frozen)
    cfg = [(3, 64), (64, 64), "M", (64, 128), (128, 128), "M", (128, 256), (256, 256),
           (256, 256), (256, 256), "M", (256, 512)]
    names = STYLE_LAYER_NAMES

    class VGGFeatures(nn.Module):
        def __init__(self):
            super().__init__()
            self.layers = nn.ModuleList()
            for c in cfg:
                if c == "M":
                    self.layers.append(nn.MaxPool2d(2))
                else:
                    self.layers.append(nn.Sequential(nn.Conv2d(c[0], c[1], 3, padding=1), nn.ReLU()))

        def forward(self, x, taps):
            out = {}
            for name, layer in zip(names, self.layers):
                x = layer(x)
                if name in taps:
                    out[name] = x
            return out

    return Generator, VGGFeatures


STYLE_LAYER_NAMES = ("relu1_1", "relu1_2", "pool1", "relu2_1", "relu2_2", "pool2", "relu3_1", "relu3_2", "relu3_3",
                     "relu3_4", "pool3", "relu4_1")
STYLE_TAPS = ("relu1_1", "relu2_1", "relu3_1", "relu4_1")
CONTENT_TAP = "relu2_2"


def gram(f):
    b, c, h, w = f.shape
    x = f.reshape(b, c, h * w)
    return (x @ x.transpose(1, 2)).float() / float(c * h * w)


def build_style(torch, device, batch=40, size=36, fused=True, region=False, lr=1e-3, weight_decay=0.0):
    """BASELINE config 4's training step on `device`; returns (step, generator).  fused:
    Adam's fused kernel (what an xdna model runs, and the reference's pre-hook picks),
    or None for the optimizer's default (single-tensor on the CPU).  region: the loss
    through xdna_train.regions.frozen_feature_loss (the frozen VGG, its content and Gram
    style terms as one fused region) and the generator's norm + ReLU pairs fused
    (regions.fuse_norm_activations); opt-in, like the reference's regions."""
    nn = torch.nn
    Generator, VGG = style_models(torch, nn)
    torch.manual_seed(0)
    gen = Generator().bfloat16()
    vgg = VGG().bfloat16()
    for p in vgg.parameters():
        p.requires_grad_(False)
    g1 = torch.Generator().manual_seed(1)
    content = torch.rand(batch, 3, size, size, generator=g1).bfloat16()
    g2 = torch.Generator().manual_seed(2)
    style = torch.rand(1, 3, size, size, generator=g2).bfloat16()
    gen.to(device)
    vgg.to(device)
    content = content.to(device)
    style = style.to(device)
    with torch.no_grad():
        sf = vgg(style, STYLE_TAPS)
        style_grams = {k: gram(v) for k, v in sf.items()}
    # capturable: the step may be captured in a graph (same fused Adam kernel either way)
    opt = torch.optim.Adam(gen.parameters(), lr=lr, weight_decay=weight_decay, fused=fused,
                           capturable=device.type != "cpu")

    if region:
        from xdna_train import regions
        regions.fuse_norm_activations(gen)  # each InstanceNorm2d + ReLU pair as one kernel pair
        flat, tap_index = [], {}
        for name, layer in zip(STYLE_LAYER_NAMES, vgg.layers):
            flat += list(layer) if isinstance(layer, torch.nn.Sequential) else [layer]
            tap_index[name] = len(flat) - 1
        chain = regions.FrozenFeatureChain.from_sequential(flat, [tap_index[k] for k in STYLE_TAPS + (CONTENT_TAP,)])
        style = {tap_index[k]: (style_grams[k], 1e5) for k in STYLE_TAPS}
        content_tap = (tap_index[CONTENT_TAP],)

        def step():
            opt.zero_grad(set_to_none=True)
            loss = regions.frozen_feature_loss(chain, gen(content), content, mse_taps=content_tap, style=style)
            loss.backward()
            opt.step()
            return loss

        return step, gen

    def step():
        opt.zero_grad(set_to_none=True)
        out = gen(content)
        with torch.no_grad():
            target = vgg(content, (CONTENT_TAP,))[CONTENT_TAP]
        feats = vgg(out, STYLE_TAPS + (CONTENT_TAP,))
        loss = torch.nn.functional.mse_loss(feats[CONTENT_TAP].float(), target.float())
        for k in STYLE_TAPS:
            g = gram(feats[k])
            loss = loss + 1e5 * torch.nn.functional.mse_loss(g, style_grams[k].expand_as(g))
        loss.backward()
        opt.step()
        return loss

    return step, gen


# ---------------------------------------------------------------------------------------
# MLP training step; config 1: one 3x3 conv
# ---------------------------------------------------------------------------------------
def build_mlp(torch, device, fused=True):
    """Linear 1024->4096->4096->1024 with GELU, x [8192,1024] and target ~ N(0,1), MSE,
    Adam 1e-3 (model seed 0, data seed 1); returns (step, model)."""
    nn = torch.nn
    torch.manual_seed(0)
    mlp = nn.Sequential(nn.Linear(1024, 4096), nn.GELU(), nn.Linear(4096, 4096), nn.GELU(),
                        nn.Linear(4096, 1024)).bfloat16().to(device)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(8192, 1024, generator=g).bfloat16().to(device)
    t = torch.randn(8192, 1024, generator=g).bfloat16().to(device)
    opt = torch.optim.Adam(mlp.parameters(), lr=1e-3, fused=fused)

    def step():
        opt.zero_grad(set_to_none=True)
        loss = torch.nn.functional.mse_loss(mlp(x).float(), t.float())
        loss.backward()
        opt.step()
        return loss

    return step, mlp


def build_c1(torch, device, fused=True):
    """BASELINE config 1 (README.md:57-68): Conv2d 128->128 3x3 pad 1 with bias, default
    init (seed 0), x ~ N(0,1) [16,128,36,36], MSE to zeros, Adam 1e-3; returns (step, conv)."""
    torch.manual_seed(0)
    conv = torch.nn.Conv2d(128, 128, 3, padding=1).bfloat16().to(device)
    x = torch.randn(16, 128, 36, 36).bfloat16().to(device)
    target = torch.zeros(16, 128, 36, 36, device=device)
    # capturable: the step may be captured in a graph (same fused Adam kernel either way)
    opt = torch.optim.Adam(conv.parameters(), lr=1e-3, fused=fused, capturable=device.type != "cpu")

    def step():
        opt.zero_grad(set_to_none=True)
        loss = torch.nn.functional.mse_loss(conv(x).float(), target)
        loss.backward()
        opt.step()
        return loss

    return step, conv


def build_resnet(torch, device, fused=True, batch=128, size=64):
    """ResNet-18-style network (BasicBlock [2,2,2,2], widths 64/128/256/
    512, 3x3 stride-1 stem, strided 3x3 + 1x1 downsample convs, BatchNorm + ReLU, global
    average pool, FC to 1000), input [128,3,64,64] ~ N(0,1), labels uniform in [0,1000),
    cross-entropy, Adam 1e-3 (model seed 0, data seed 1); returns (step, model)."""
    nn = torch.nn

    class Block(nn.Module):
        def __init__(self, cin, cout, stride):
            super().__init__()
            self.c1 = nn.Conv2d(cin, cout, 3, stride, 1, bias=False)
            self.b1 = nn.BatchNorm2d(cout)
            self.c2 = nn.Conv2d(cout, cout, 3, 1, 1, bias=False)
            self.b2 = nn.BatchNorm2d(cout)
            self.down = None
            if stride != 1 or cin != cout:
                self.down = nn.Sequential(nn.Conv2d(cin, cout, 1, stride, bias=False), nn.BatchNorm2d(cout))

        def forward(self, x):
            y = torch.relu(self.b1(self.c1(x)))
            y = self.b2(self.c2(y))
            return torch.relu(y + (x if self.down is None else self.down(x)))

    class ResNet18(nn.Module):
        def __init__(self):
            super().__init__()
            self.stem = nn.Sequential(nn.Conv2d(3, 64, 3, 1, 1, bias=False), nn.BatchNorm2d(64), nn.ReLU())
            blocks, cin = [], 64
            for cout, stride in ((64, 1), (128, 2), (256, 2), (512, 2)):
                blocks += [Block(cin, cout, stride), Block(cout, cout, 1)]
                cin = cout
            self.blocks = nn.Sequential(*blocks)
            self.pool = nn.AdaptiveAvgPool2d(1)
            self.fc = nn.Linear(512, 1000)

        def forward(self, x):
            return self.fc(torch.flatten(self.pool(self.blocks(self.stem(x))), 1))

    torch.manual_seed(0)
    model = ResNet18().bfloat16().to(device).train()
    g = torch.Generator().manual_seed(1)
    x = torch.randn(batch, 3, size, size, generator=g).bfloat16().to(device)
    labels = torch.randint(0, 1000, (batch,), generator=g).to(device)
    opt = torch.optim.Adam(model.parameters(), lr=1e-3, fused=fused)

    def step():
        opt.zero_grad(set_to_none=True)
        loss = torch.nn.functional.cross_entropy(model(x).float(), labels)
        loss.backward()
        opt.step()
        return loss

    return step, model


RESNET_GFLOP = 3 * 2 * 284.4  # fwd + dgrad + wgrad of its 284.4 GMAC forward (dgrad of the stem included)


# ---------------------------------------------------------------------------------------
def sync(torch):
    torch.xdna.synchronize()


def conv_sweep_data(torch, device, shapes, first_index=0):
    """x, w, b, dy of each shape; shape i of the sweep is seeded 1000 + i (`first_index`
    names the sweep index of shapes[0])."""
    data = []
    for idx, (n, c, h) in enumerate(shapes, start=first_index):
        torch.manual_seed(1000 + idx)
        bound = math.sqrt(6.0 / (9 * c))
        x = torch.randn(n, c, h, h, device=device).bfloat16()
        w = ((torch.rand(c, c, 3, 3, device=device) * 2 - 1) * bound).bfloat16().requires_grad_()
        b = ((torch.rand(c, device=device) * 2 - 1) / math.sqrt(9 * c)).bfloat16()
        dy = torch.randn(n, c, h, h, device=device).bfloat16()
        data.append((x, w, b, dy))
    return data


def conv_step(torch, data, note_write=None):
    """fwd + dgrad + wgrad (+ bias grad) of every shape through the aten ops.  note_write:
    called on each weight first, recording a write as the optimizer step of a training
    step makes, so the weight's prepared forms are made again (as in training); None leaves
    the weights unwritten, so the forms cached by the previous step serve.  no_grad: the
    aten calls are the whole step, nothing is recorded for autograd."""
    aten = torch.ops.aten
    s, p, d, op = [1, 1], [1, 1], [1, 1], [0, 0]
    with torch.no_grad():
        for x, w, b, dy in data:
            if note_write is not None:
                note_write(w)
            aten.convolution_overrideable(x, w, b, s, p, d, False, op, 1)
            aten.convolution_backward_overrideable(dy, x, w, s, p, d, False, op, 1, [True, True, True])


def sweep_flops(shapes):
    return sum(3 * 2.0 * n * h * h * c * c * 9 for n, c, h in shapes)


# ---------------------------------------------------------------------------------------
# CPU baseline: the reference's CPU BF16 path (stock PyTorch CPU kernels) timed on this
# box's host cores, in worker processes alternating with the GPU timing of the same
# workload (ABBA over rounds), median of the per-round medians (the reference's method,
# benchmarks/end_to_end_speed.py:53-64, 98-107 and model_zoo.py:281-286).
# ---------------------------------------------------------------------------------------
# every C and H of the sweep at N16: the sample the CPU conv rate is measured on
CPU_SWEEP_SAMPLE = [(16, c, h) for c in (64, 128, 256, 512) for h in (18, 36, 72)]


def cpu_topology():
    """(cpus in this process's affinity, physical cores among them, lscpu model name)."""
    aff = sorted(os.sched_getaffinity(0))
    cores = set()
    for cpu in aff:
        try:
            base = f"/sys/devices/system/cpu/cpu{cpu}/topology/"
            cores.add((open(base + "physical_package_id").read().strip(), open(base + "core_id").read().strip()))
        except OSError:
            cores.add(("cpu", str(cpu)))
    model = ""
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        model = next((ln.split(":", 1)[1].strip() for ln in out.splitlines() if ln.startswith("Model name")), "")
    except (OSError, ValueError):
        pass
    return len(aff), len(cores), model


def cpu_threads():
    """Physical cores visible to the process, capped by the box's CPU share (OMP_NUM_THREADS)."""
    _, phys, _ = cpu_topology()
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return max(1, min(phys, share) if share > 0 else phys)


def timed_steps(step, warmup, steps, sync_fn):
    """Per-step wall times (s) of `steps` steps after `warmup`; each step ends in a host read
    of its result, as a logging script does (end_to_end_speed.py:53-64)."""
    for _ in range(warmup):
        step()
    sync_fn()
    times = []
    for _ in range(steps):
        t0 = time.perf_counter()
        out = step()
        if out is not None:
            float(out.detach())
        sync_fn()
        times.append(time.perf_counter() - t0)
    return times


def sweep_sample_step(torch, device):
    """One fwd + dgrad + wgrad (+ bias grad) pass over CPU_SWEEP_SAMPLE through
    F.conv2d and autograd (the reference's CPU path; on xdna the same aten ops)."""
    data = conv_sweep_data(torch, device, CPU_SWEEP_SAMPLE)

    def step():
        for x, w, b, dy in data:
            xr = x.detach().requires_grad_()
            wr = w.detach().requires_grad_()
            br = b.detach().requires_grad_()
            torch.nn.functional.conv2d(xr, wr, br, padding=1).backward(dy)
        return None

    return step


CPU_WORKLOADS = {
    # name -> (builder(torch, device) -> step, warmup, steps, unit, work per step)
    "conv_sweep_sample": (lambda t, d: sweep_sample_step(t, d), 1, 3, "TFLOP/s", sweep_flops(CPU_SWEEP_SAMPLE)),
    "c1_default_adam": (lambda t, d: build_c1(t, d, fused=None)[0], 3, 20, "it/s", 1.0),
    "style_default_adam": (lambda t, d: build_style(t, d, fused=None)[0], 3, 20, "it/s", 1.0),
    "style_fused_adam": (lambda t, d: build_style(t, d, fused=True)[0], 3, 20, "it/s", 1.0),
    "resnet18_default_adam": (lambda t, d: build_resnet(t, d, fused=None)[0], 2, 5, "it/s", 1.0),
}


def cpu_worker(name):
    """Runs one CPU workload in this (fresh) process and prints RESULT={json}."""
    import torch

    threads = cpu_threads()
    torch.set_num_threads(threads)
    build, warmup, steps, unit, work = CPU_WORKLOADS[name]
    step = build(torch, torch.device("cpu"))
    times = timed_steps(step, warmup, steps, lambda: None)
    med = statistics.median(times)
    rate = work / med / (1e12 if unit == "TFLOP/s" else 1.0)
    print("RESULT=" + json.dumps({"name": name, "median_s": med, "rate": rate, "unit": unit, "steps": steps,
                                  "threads": threads}), flush=True)


def run_cpu_worker(name, timeout=600):
    import subprocess
    env = dict(os.environ, XDNA_CPU_WORKER="1")
    p = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-worker", name], capture_output=True,
                       text=True, env=env, timeout=timeout)
    for ln in p.stdout.splitlines():
        if ln.startswith("RESULT="):
            return json.loads(ln[7:])
    raise RuntimeError(f"cpu worker {name} failed (rc {p.returncode}):\n{p.stderr[-2000:]}")


def abba(cpu_name, gpu_rate, rounds=2, log=None):
    """ABBA rounds of the CPU worker and the GPU timing (gpu_rate() -> rate in the worker's
    unit); medians over the rounds."""
    cpu, gpu = [], []
    for r in range(rounds):
        for side in (("cpu", "gpu") if r % 2 == 0 else ("gpu", "cpu")):
            if side == "cpu":
                cpu.append(run_cpu_worker(cpu_name)["rate"])
            else:
                gpu.append(gpu_rate())
        if log:
            log(f"cpu baseline {cpu_name}: round {r + 1}: cpu {cpu[-1]:.4g}, gpu {gpu[-1]:.4g}")
    return statistics.median(cpu), statistics.median(gpu), cpu, gpu


CALIB_BYTES = 256 << 20     # plain device copy whose PMC byte counts calibrate FETCH/WRITE_SIZE
TRAFFIC_FILE = REPO / "profiles" / "conv_sweep_hbm_traffic.json"


def calibration_copy(torch, C):
    """One D2D copy of CALIB_BYTES through the C ABI (hipMemcpyAsync's blit kernel): the
    reference kernel of known size for the rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs."""
    from xdna_train import hip_abi
    lib = hip_abi.load()
    src = torch.empty(CALIB_BYTES, dtype=torch.uint8, device="xdna")
    dst = torch.empty_like(src)
    rc = lib.xdna_hip_memcpy_async(C.data_ptr(dst), C.data_ptr(src), CALIB_BYTES, 3,
                                   torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    sync(torch)


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed PMC summary (two rocprofv3 --pmc
    runs of this script over the sweep, FETCH_SIZE then WRITE_SIZE, each scaled by the
    calibration copy's reading), or None."""
    try:
        d = json.loads(TRAFFIC_FILE.read_text())
        return d["kernels"][kernel]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def kernel_summary(report):
    out = {}
    for name, e in report.items():
        ms = e["total_ms"]
        rate = e["work"] / (ms * 1e-3) if ms > 0 else 0.0
        is_bytes = name in ("conv3x3w_pack", "fused_adam", "conv3x3_prep")
        out[name] = {"launches": e["launches"], "total_ms": round(ms, 4),
                     "avg_us": round(1e3 * ms / max(1, e["launches"]), 3),
                     ("GB/s" if is_bytes else "TFLOP/s"): round(rate / (1e9 if is_bytes else 1e12), 2)}
    return out


def shape_table(torch, C, X, reps=5, cpu=True, log=None):
    """Per-shape figures of the sweep (the reference's per-shape report of config 2,
    benchmarks/conv_shape_sweep.py:60-126): each shape's fwd + dgrad + wgrad step with its
    weight written first (wall time over `reps` steps), the kernel time of every direction
    (HIP events on the launch stream) as TFLOP/s and a fraction of the dense bf16 peak, the
    packs' and weight preparations' GB/s, and the CPU bf16 path per direction (torch CPU,
    the same operands, one warm-up and the median of three runs each)."""
    import torch.nn.functional as F
    rows = []
    threads = cpu_threads()
    for idx, (n, c, h) in enumerate(SWEEP):
        data = conv_sweep_data(torch, X, [(n, c, h)], first_index=idx)
        for _ in range(2):
            conv_step(torch, data, C.note_write)
        sync(torch)
        t0 = time.perf_counter()
        for _ in range(reps):
            conv_step(torch, data, C.note_write)
        sync(torch)
        wall = (time.perf_counter() - t0) / reps
        C.kernel_timing(True)
        for _ in range(reps):
            conv_step(torch, data, C.note_write)
        rep = dict(C.kernel_timing_report())
        C.kernel_timing(False)
        flop = 2.0 * n * h * h * c * c * 9
        e = {"N": n, "C": c, "H": h, "gflop_per_direction": round(flop / 1e9, 3), "step_us": round(1e6 * wall, 1),
             "step_tflops": round(3 * flop / wall / 1e12, 1)}
        for key, name in (("fwd", "conv3x3_rows.fwd"), ("dgrad", "conv3x3_rows.dgrad"), ("wgrad", "conv3x3_wgrad")):
            k = rep.get(name)
            if k:
                us = 1e3 * k["total_ms"] / k["launches"]
                e[key + "_us"] = round(us, 1)
                e[key + "_tflops"] = round(flop / (us * 1e-6) / 1e12, 1)
                e[key + "_frac_peak"] = round(flop / (us * 1e-6) / 1e12 / PEAK_BF16_TFLOPS, 4)
        for key, name in (("pack", "conv3x3w_pack"), ("prep", "conv3x3_prep")):
            k = rep.get(name)
            if k:
                e[key + "_us"] = round(1e3 * k["total_ms"] / k["launches"], 2)
                e[key + "_gbs"] = round(k["work"] / (k["total_ms"] * 1e-3) / 1e9, 1)
        if cpu:
            torch.set_num_threads(threads)
            x, w, b, dy = (t.detach().cpu() for t in data[0])
            aten = torch.ops.aten

            def cpu_ms(fn):
                fn()
                ts = []
                for _ in range(3):
                    t1 = time.perf_counter()
                    fn()
                    ts.append(time.perf_counter() - t1)
                return 1e3 * statistics.median(ts)

            e["cpu_fwd_ms"] = round(cpu_ms(lambda: F.conv2d(x, w, b, padding=1)), 2)
            e["cpu_dgrad_ms"] = round(cpu_ms(lambda: aten.convolution_backward(
                dy, x, w, None, [1, 1], [1, 1], [1, 1], False, [0, 0], 1, [True, False, False])), 2)
            e["cpu_wgrad_ms"] = round(cpu_ms(lambda: aten.convolution_backward(
                dy, x, w, [c], [1, 1], [1, 1], [1, 1], False, [0, 0], 1, [False, True, True])), 2)
        rows.append(e)
        del data
        if log:
            log(f"shape {n} {c} {h}: {e['step_tflops']} TFLOP/s")
    return {"shapes": rows, "reps": reps, "cpu_threads": threads if cpu else None,
            "cpu_model": cpu_topology()[2] if cpu else None}


def gemm_product(layout, variant, M=8192, N=4096, K=4096, launches=30):
    """Launches one config-3 product through the C ABI with a forced kernel variant: the
    workload of the GEMM counter passes (rocprofv3 --pmc)."""
    import torch

    from xdna_train import hip_abi
    lib = hip_abi.load()
    st = torch.cuda.current_stream().cuda_stream
    g = torch.Generator().manual_seed(0)
    a = (torch.randn(K, M, generator=g) if layout[0] == "t" else torch.randn(M, K, generator=g)).cuda().bfloat16()
    b = (torch.randn(N, K, generator=g) if layout[1] == "t" else torch.randn(K, N, generator=g)).cuda().bfloat16()
    a_s = (1, M) if layout[0] == "t" else (K, 1)
    b_s = (1, K) if layout[1] == "t" else (N, 1)
    c = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    assert lib.xdna_gemm_set_variant(int(variant)) == 0
    for _ in range(launches):
        assert lib.xdna_gemm_bf16(a.data_ptr(), b.data_ptr(), c.data_ptr(), None, 1, M, N, K, a_s[0], a_s[1], 0,
                                  b_s[0], b_s[1], 0, N, 1, M * N, 0, 0, 1, 1.0, 0.0, st) == 0
    torch.cuda.synchronize()
    print(f"gemm product {layout} variant {variant}: {launches} launches", flush=True)
    return 0


def conv_rows_shape(variant, n, c, h, launches=20):
    """20 forward 3x3 convs of one sweep-shaped problem (N, C, H = W; seeded sweep data) through
    the aten op with xdna_conv3x3_set_rows_variant VARIANT: the workload of the rows-kernel
    counter passes (rocprofv3 --pmc)."""
    import torch

    import xdna_train  # noqa: F401  (registers the xdna device)
    from xdna_train import hip_abi
    lib = hip_abi.load()
    X = torch.device("xdna")
    (x, w, b, _), = conv_sweep_data(torch, X, [(int(n), int(c), int(h))])
    assert lib.xdna_conv3x3_set_rows_variant(int(variant)) == 0
    with torch.no_grad():
        for _ in range(launches):
            torch.ops.aten.convolution_overrideable(x, w, b, [1, 1], [1, 1], [1, 1], False, [0, 0], 1)
    sync(torch)
    assert lib.xdna_conv3x3_set_rows_variant(0) == 0
    print(f"conv rows variant {variant} N{n} C{c} H{h}: {launches} forward convs", flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--style-steps", type=int, default=20)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-style", action="store_true")
    ap.add_argument("--skip-mlp", action="store_true")
    ap.add_argument("--mlp-steps", type=int, default=10)
    ap.add_argument("--quick", action="store_true", help="small subset (profiling runs)")
    ap.add_argument("--skip-resnet", action="store_true")
    ap.add_argument("--skip-c1", action="store_true")
    ap.add_argument("--c1-steps", type=int, default=50)
    ap.add_argument("--shape-table", action="store_true",
                    help="per-shape fwd / dgrad / wgrad / pack figures of the sweep (GPU kernel times and "
                         "the CPU bf16 path per direction), one JSON object")
    ap.add_argument("--resnet-steps", type=int, default=10)
    ap.add_argument("--cpu-rounds", type=int, default=2)
    ap.add_argument("--cpu-worker", help=argparse.SUPPRESS)
    ap.add_argument("--gemm-product", metavar="LAYOUT,VARIANT",
                    help="only 30 launches of config 3's largest product (M 8192, N 4096, K 4096) with "
                         "operand layout nt / nn / tn and xdna_gemm_set_variant VARIANT (counter passes)")
    ap.add_argument("--conv-rows", metavar="VARIANT,N,C,H",
                    help="only 20 forward convs of one sweep shape with xdna_conv3x3_set_rows_variant "
                         "VARIANT (counter passes)")
    args = ap.parse_args()
    if args.cpu_worker:
        cpu_worker(args.cpu_worker)
        return 0
    if args.gemm_product:
        return gemm_product(*args.gemm_product.split(","))
    if args.conv_rows:
        return conv_rows_shape(*args.conv_rows.split(","))
    if args.gpus != 1:
        print("bench.py: this build runs on one MI355X only (one process, one GPU); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        return 2

    import torch

    import xdna_train

    assert xdna_train.is_available(), "xdna device not available"
    from xdna_train import device as xdev

    C = xdev.native()
    X = torch.device("xdna")
    log = lambda *a: print("[bench]", *a, file=sys.stderr, flush=True)  # noqa: E731
    if args.shape_table:
        print(json.dumps(shape_table(torch, C, X, cpu=not args.skip_cpu, log=log)), flush=True)
        return 0

    calibration_copy(torch, C)

    # --- headline: conv sweep --------------------------------------------------------
    shapes = SWEEP if not args.quick else [(16, 128, 36), (64, 256, 36)]
    log(f"conv sweep: {len(shapes)} shapes, building data")
    data = conv_sweep_data(torch, X, shapes)
    # every step writes the weights first (as an optimizer step does), so each step prepares
    # every weight's forms again, as in training
    note = C.note_write
    for _ in range(args.warmup):
        conv_step(torch, data, note)
    sync(torch)
    log("conv sweep: warm")
    # value: K steps with nothing but the step on the stream
    sync(torch)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        conv_step(torch, data, note)
    sync(torch)
    dt = time.perf_counter() - t0
    flops_step = sweep_flops(shapes)
    value = flops_step * args.steps / dt / 1e12
    log(f"conv sweep: {value:.1f} TFLOP/s, {1e3 * dt / args.steps:.2f} ms/step")
    # beside it: the same steps with the weights unwritten (their prepared forms cached)
    sync(torch)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        conv_step(torch, data)
    sync(torch)
    dt_cached = time.perf_counter() - t0
    # per-kernel figures (and the roofline): K more steps with a HIP event pair around every
    # hot-kernel launch.  The event records cost GPU time between launches, so this pass
    # is not the one `value` is timed on.
    C.kernel_timing(True)
    sync(torch)
    t1 = time.perf_counter()
    for _ in range(args.steps):
        conv_step(torch, data, note)
    sync(torch)
    dt_ev = time.perf_counter() - t1
    kreport = dict(C.kernel_timing_report())
    C.kernel_timing(False)
    kernels = kernel_summary(kreport)
    log(f"conv sweep with per-kernel events: {1e3 * dt_ev / args.steps:.2f} ms/step")

    # dominant kernel of the timed region (largest total time among the MFMA kernels)
    groups = {"conv3x3_rows": ["conv3x3_rows.fwd", "conv3x3_rows.dgrad"], "conv3x3_wgrad": ["conv3x3_wgrad"]}
    tot = {g: sum(kreport.get(n, {}).get("total_ms", 0.0) for n in ns) for g, ns in groups.items()}
    dom = max(tot, key=tot.get)
    work = sum(kreport.get(n, {}).get("work", 0.0) for n in groups[dom])
    launches = sum(kreport.get(n, {}).get("launches", 0) for n in groups[dom])
    achieved = work / (tot[dom] * 1e-3) / 1e12
    roofline = {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 2),
                "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                "traffic": measured_traffic(dom) if not args.quick else None, "launches": launches,
                "avg_launch_us": round(1e3 * tot[dom] / max(1, launches), 3),
                "flop_per_launch_avg": work / max(1, launches)}
    per_dir = {}
    for name in ("conv3x3_rows.fwd", "conv3x3_rows.dgrad", "conv3x3_wgrad"):
        e = kreport.get(name)
        if e:
            per_dir[name] = round(e["work"] / (e["total_ms"] * 1e-3) / 1e12, 1)

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * dt / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations and dY, Kaiming-uniform weights)",
        "config": {"workload": "BASELINE config 2: 3x3 conv sweep, stride 1, pad 1, bias, bf16, "
                               "N{16,40,64} x C{64,128,256,512} x H=W{18,36,72}; step = fwd + dgrad + "
                               "wgrad(+bias grad) of every shape via aten convolution(_backward)_overrideable, "
                               "each weight written first (its forms prepared every step, as in training)",
                   "shapes": len(shapes), "gflop_per_step": round(flops_step / 1e9, 1),
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "weights_unwritten": {"TFLOP/s": round(flops_step * args.steps / dt_cached / 1e12, 2),
                              "ms_per_step": round(1e3 * dt_cached / args.steps, 3),
                              "note": "the same steps without the per-step weight write: every weight's "
                                      "prepared forms come from the cache"},
        "kernel_timing_pass_ms_per_step": round(1e3 * dt_ev / args.steps, 3),
        "kernel_tflops_by_direction": per_dir,
        "kernels": kernels,
    }

    # --- fused Adam at config 3's parameter count --------------------------------------
    params = [torch.nn.Parameter(torch.randn(ADAM_PARAMS, device=X).bfloat16())]
    params[0].grad = (torch.randn(ADAM_PARAMS, device=X) * 1e-2).bfloat16()
    opt = torch.optim.Adam(params, lr=1e-3, fused=True)
    for _ in range(3):
        opt.step()
    sync(torch)
    C.kernel_timing(True)
    for _ in range(10):
        opt.step()
    ar = dict(C.kernel_timing_report()).get("fused_adam", {})
    C.kernel_timing(False)
    if ar:
        gbs = ar["work"] / (ar["total_ms"] * 1e-3) / 1e9
        result["adam"] = {"params": ADAM_PARAMS, "bytes_per_param": 14, "GB/s": round(gbs, 1),
                          "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
                          "avg_launch_us": round(1e3 * ar["total_ms"] / ar["launches"], 2)}
        log(f"adam: {gbs:.0f} GB/s")
    del params, opt

    # --- config 1: one Conv2d(128->128) training step --------------------------------------
    if not args.skip_c1:
        log("c1: building")
        c1_step, _ = build_c1(torch, X)
        c1_eager = 1.0 / statistics.median(timed_steps(c1_step, 3, args.c1_steps, lambda: sync(torch)))
        c1_graph = xdna_train.Graph()
        with xdna_train.graph(c1_graph):
            c1_loss = c1_step()
        for _ in range(2):
            c1_graph.replay()
        sync(torch)
        t0 = time.perf_counter()
        for _ in range(args.c1_steps):
            c1_graph.replay()
        float(c1_loss.detach())
        c1_it_s = args.c1_steps / (time.perf_counter() - t0)
        c1_graph.reset()
        C.kernel_timing(True)
        for _ in range(args.c1_steps):
            c1_step()
        c1rep = dict(C.kernel_timing_report())
        C.kernel_timing(False)
        # forward and weight gradient (x is data: no input gradient is computed)
        c1_flop = 2.0 * 16 * 36 * 36 * 128 * 128 * 9
        c1_dirs = {}
        for key, name in (("fwd", "conv3x3_rows.fwd"), ("dgrad", "conv3x3_rows.dgrad"), ("wgrad", "conv3x3_wgrad")):
            e = c1rep.get(name)
            if e:
                tf = e["work"] / (e["total_ms"] * 1e-3) / 1e12
                c1_dirs[key] = {"TFLOP/s": round(tf, 1), "frac_peak": round(tf / PEAK_BF16_TFLOPS, 4),
                                "avg_us": round(1e3 * e["total_ms"] / e["launches"], 2)}
        ea = c1rep.get("fused_adam")
        c1_adam = None
        if ea:
            gb = ea["work"] / (ea["total_ms"] * 1e-3) / 1e9
            c1_adam = {"params": 147584, "GB/s": round(gb, 1), "frac_hbm": round(gb / PEAK_HBM_GBS, 4),
                       "avg_us": round(1e3 * ea["total_ms"] / ea["launches"], 2)}
        result["c1"] = {"it_s": round(c1_it_s, 1), "mode": "HIP graph replay of the whole training step",
                        "eager_it_s": round(c1_eager, 1), "gflop_per_step": round(2 * c1_flop / 1e9, 2),
                        "step_tflops": round(2 * c1_flop * c1_it_s / 1e12, 1), "by_direction": c1_dirs,
                        "adam": c1_adam,
                        "workload": "BASELINE config 1: Conv2d 128->128 3x3 pad 1 + bias, x [16,128,36,36], "
                                    "MSE to zeros, Adam 1e-3 (README.md:57-68); fwd + wgrad (+ bias grad) per "
                                    "step, x needs no gradient"}
        log(f"c1: {c1_it_s:.1f} it/s (graph), {c1_eager:.1f} it/s (eager)")

        def c1_gpu_it_s():
            return 1.0 / statistics.median(timed_steps(c1_step, 3, args.c1_steps, lambda: sync(torch)))

    # --- MLP training step (config 3): mm / addmm fwd + both backward GEMMs + Adam -------
    if not args.skip_mlp:
        log("mlp: building")
        mlp_step, _ = build_mlp(torch, X)

        for _ in range(3):
            mlp_step()
        sync(torch)
        C.kernel_timing(True)
        t0 = time.perf_counter()
        for _ in range(args.mlp_steps):
            mloss = mlp_step()
        sync(torch)
        dtm = time.perf_counter() - t0
        mrep = dict(C.kernel_timing_report())
        C.kernel_timing(False)
        # fwd 3 GEMMs + dW 3 + dX 2 (the input needs no gradient): 2*T*(sum of in*out) each
        gemm_flop = 2.0 * 8192 * (1024 * 4096 + 4096 * 4096 + 4096 * 1024) * 3 - 2.0 * 8192 * 1024 * 4096
        ge = mrep.get("gemm", {})
        result["mlp"] = {
            "steps": args.mlp_steps, "ms_per_step": round(1e3 * dtm / args.mlp_steps, 3),
            "step_gemm_tflops": round(gemm_flop * args.mlp_steps / dtm / 1e12, 1),
            "gemm_kernel_tflops": round(ge["work"] / (ge["total_ms"] * 1e-3) / 1e12, 1) if ge else None,
            "gemm_launches_per_step": ge.get("launches", 0) // max(1, args.mlp_steps),
            "loss": float(mloss.item()),
            "workload": "BASELINE config 3: Linear 1024->4096->4096->1024, GELU, bias, x [8192,1024], MSE, Adam; "
                        "step_gemm_tflops = 1168.2 GFLOP of GEMM per step / wall time of the whole step",
        }
        log(f"mlp: {result['mlp']['ms_per_step']} ms/step, {result['mlp']['step_gemm_tflops']} TFLOP/s")
        del mlp_step

    # --- style step (config 4) ---------------------------------------------------------
    if not args.skip_style:
        log("style net: building")
        step, _ = build_style(torch, X)
        for _ in range(3):
            step()
        sync(torch)
        t0 = time.perf_counter()
        for _ in range(args.style_steps):
            loss = step()
        loss.item()
        dts = time.perf_counter() - t0
        eager_it_s = args.style_steps / dts
        log(f"style net (eager): {eager_it_s:.1f} it/s")
        # the same step captured once as a HIP graph and replayed (no per-op host work)
        graph = xdna_train.Graph()
        with xdna_train.graph(graph):
            gloss = step()
        for _ in range(2):
            graph.replay()
        sync(torch)
        t0 = time.perf_counter()
        for _ in range(args.style_steps):
            graph.replay()
        loss_g = float(gloss.item())
        dtg = time.perf_counter() - t0
        it_s = args.style_steps / dtg
        result["style_net"] = {"it_s": round(it_s, 2), "mode": "HIP graph replay of the whole training step",
                               "ms_per_step": round(1e3 * dtg / args.style_steps, 3),
                               "eager_it_s": round(eager_it_s, 2),
                               "eager_ms_per_step": round(1e3 * dts / args.style_steps, 3),
                               "steps": args.style_steps, "loss": loss_g}
        log(f"style net (graph): {it_s:.1f} it/s, loss {loss_g:.4f}")
        graph.reset()

        # the same step with the loss as one fused frozen-feature region (opt-in, as the
        # reference's "XDNA + fused loss region" figure)
        rstep, _ = build_style(torch, X, region=True)
        for _ in range(3):
            rstep()
        sync(torch)
        rgraph = xdna_train.Graph()
        with xdna_train.graph(rgraph):
            rloss = rstep()
        for _ in range(2):
            rgraph.replay()
        sync(torch)
        t0 = time.perf_counter()
        for _ in range(args.style_steps):
            rgraph.replay()
        r_loss = float(rloss.item())
        r_it_s = args.style_steps / (time.perf_counter() - t0)
        rgraph.reset()
        result["style_net"]["region_it_s"] = round(r_it_s, 2)
        result["style_net"]["region_ms_per_step"] = round(1e3 / r_it_s, 3)
        result["style_net"]["region_loss"] = r_loss
        result["style_net"]["region"] = ("loss via xdna_train.regions.frozen_feature_loss (frozen VGG conv+ReLU "
                                         "epilogues, device-side tap terms, fused backward), HIP graph replay")
        log(f"style net (region, graph): {r_it_s:.1f} it/s, loss {r_loss:.4f}")
        del rstep

        def style_gpu_it_s():
            g2 = xdna_train.Graph()
            with xdna_train.graph(g2):
                l2 = step()
            g2.replay()
            sync(torch)
            t1 = time.perf_counter()
            for _ in range(args.style_steps):
                g2.replay()
            float(l2.detach())
            rate = args.style_steps / (time.perf_counter() - t1)
            g2.reset()
            return rate

    # --- ResNet-18 training step (config 5) --------------------------------------------
    if not args.skip_resnet:
        log("resnet18: building")
        rstep, _ = build_resnet(torch, X)
        rt = timed_steps(rstep, 3, args.resnet_steps, lambda: sync(torch))
        r_it_s = 1.0 / statistics.median(rt)
        result["resnet18"] = {"it_s": round(r_it_s, 2), "ms_per_step": round(1e3 * statistics.median(rt), 3),
                              "mode": "eager", "steps": args.resnet_steps,
                              "step_tflops": round(RESNET_GFLOP * r_it_s / 1e3, 1),
                              "workload": "BASELINE config 5: ResNet-18 (BasicBlock [2,2,2,2]), B128 3x64x64, "
                                          "CE, Adam; median step time, each step ending in loss.item()"}
        log(f"resnet18: {r_it_s:.1f} it/s")

        # --- CPU baselines (the reference's CPU BF16 path), ABBA against the GPU ------------
    if not args.skip_cpu:
        n_aff, n_phys, model = cpu_topology()
        threads = cpu_threads()
        log(f"cpu baseline: {threads} threads ({n_phys} physical cores of {n_aff} CPUs visible; {model})")
        sample_step = sweep_sample_step(torch, X)
        sample_flops = sweep_flops(CPU_SWEEP_SAMPLE)

        def sweep_sample_gpu_tflops():
            ts = timed_steps(sample_step, 1, 5, lambda: sync(torch))
            return sample_flops / statistics.median(ts) / 1e12

        c_tf, g_tf, c_runs, g_runs = abba("conv_sweep_sample", sweep_sample_gpu_tflops, args.cpu_rounds, log)
        result["cpu_baseline"] = {
            "value": round(c_tf, 4), "unit": "TFLOP/s", "cores": threads, "kind": "reference",
            "sample": f"PyTorch CPU bf16 conv2d fwd+dgrad+wgrad(+bias grad) (the reference's CPU BF16 path) over "
                      f"{len(CPU_SWEEP_SAMPLE)} sweep shapes, N16 x every C {{64..512}} x every H {{18,36,72}} "
                      f"({sample_flops / 1e9:.0f} GFLOP per pass), median of 3 passes per worker",
            "method": f"separate worker processes, ABBA over {args.cpu_rounds} rounds against the GPU timing of the "
                      f"same sample, median of per-round medians",
            "cpu_rounds": [round(v, 4) for v in c_runs], "gpu_same_sample_tflops": round(g_tf, 1),
            "gpu_rounds": [round(v, 1) for v in g_runs], "speedup_same_sample": round(g_tf / c_tf, 1),
            "threads": threads, "physical_cores_visible": n_phys, "cpus_in_affinity": n_aff, "cpu_model": model,
        }
        log(f"cpu baseline: conv sample {c_tf:.3f} TFLOP/s on the CPU, {g_tf:.1f} on the GPU")
        if "c1" in result:
            c_c1, g_c1, cc1_runs, gc1_runs = abba("c1_default_adam", c1_gpu_it_s, args.cpu_rounds, log)
            result["c1"].update({"cpu_it_s": round(c_c1, 2), "cpu_it_s_rounds": [round(v, 2) for v in cc1_runs],
                                 "gpu_eager_it_s_abba": round(g_c1, 1),
                                 "speedup_vs_cpu": round(result["c1"]["it_s"] / c_c1, 1),
                                 "eager_speedup_vs_cpu": round(g_c1 / c_c1, 1)})
            log(f"c1 CPU: {c_c1:.2f} it/s")
        if "style_net" in result:
            c_d, g_d, cd_runs, gd_runs = abba("style_default_adam", style_gpu_it_s, args.cpu_rounds, log)
            c_f, _, cf_runs, _ = abba("style_fused_adam", style_gpu_it_s, 1, log)
            result["style_net"].update({
                "cpu_it_s": round(c_d, 3), "cpu_it_s_rounds": [round(v, 3) for v in cd_runs],
                "cpu_adam": "CPU default (single-tensor) Adam, the reference's CPU path",
                "cpu_fused_adam_it_s": round(c_f, 3), "gpu_it_s_abba": round(g_d, 2),
                "gpu_it_s_abba_rounds": [round(v, 2) for v in gd_runs],
                "speedup_vs_cpu": round(result["style_net"]["it_s"] / c_d, 1),
                "eager_speedup_vs_cpu": round(result["style_net"]["eager_it_s"] / c_d, 1),
                "speedup_vs_cpu_fused_adam": round(result["style_net"]["it_s"] / c_f, 1)})
            if "region_it_s" in result["style_net"]:
                result["style_net"]["region_speedup_vs_cpu"] = round(result["style_net"]["region_it_s"] / c_d, 1)
            log(f"style net CPU: {c_d:.2f} it/s (default Adam), {c_f:.2f} it/s (fused Adam)")
        if "resnet18" in result:
            c_r, g_r, cr_runs, gr_runs = abba(
                "resnet18_default_adam",
                lambda: 1.0 / statistics.median(timed_steps(rstep, 1, args.resnet_steps, lambda: sync(torch))),
                args.cpu_rounds, log)
            result["resnet18"].update({"cpu_it_s": round(c_r, 3), "cpu_it_s_rounds": [round(v, 3) for v in cr_runs],
                                       "gpu_it_s_abba": round(g_r, 2),
                                       "speedup_vs_cpu": round(result["resnet18"]["it_s"] / c_r, 1)})
            log(f"resnet18 CPU: {c_r:.3f} it/s")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
