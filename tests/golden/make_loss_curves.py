"""Writes tests/golden/loss_curves.json: 200-step CPU bf16 loss curves of BASELINE configs
3 (MLP) and 5 (ResNet-18), the reference's CPU BF16 path (stock PyTorch CPU kernels, the
same seeded builds as bench.py), for the GPU loss-curve tests to compare against.

Per config: the fused-Adam run (what the reference executes for an xdna model: its
pre-hook picks fused=True and the CPU kernel runs it), the default single-tensor Adam run,
and three runs whose only difference is one weight moved by one bf16 ulp (the CPU's own
rounding spread; same rule as tests/test_gpu_loss_curves.py:_nudge).  Computed once in the
build container because five 200-step CPU runs of these configs do not fit a GPU test's
time budget; the torch version, thread count and CPU model are recorded beside them.

    python tests/golden/make_loss_curves.py [--steps 200] [--configs c3,c5]
"""
from __future__ import annotations

import argparse
import json
import platform
import sys
import time
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path.insert(0, str(REPO))
sys.path.insert(0, str(REPO / "tests"))

import torch  # noqa: E402

import bench  # noqa: E402

BUILDS = {"c3": bench.build_mlp, "c5": bench.build_resnet}


def nudge(model, where):
    """Moves one element of the first trainable weight by one bf16 ulp (element 0, the
    middle one or the last one)."""
    p = next(q for q in model.parameters() if q.requires_grad and q.numel() > 1)
    flat = p.data.view(-1)
    i = [0, flat.numel() // 2, flat.numel() - 1][where]
    with torch.no_grad():
        v = flat[i:i + 1].float()
        flat[i:i + 1] = (v * (1 + 2.0 ** -7)).bfloat16()


def curve(build, steps, fused, where=None):
    step, model = build(torch, torch.device("cpu"), fused=fused)
    if where is not None:
        nudge(model, where)
    out = []
    for i in range(steps):
        out.append(float(step().detach()))
        if i % 50 == 49:
            print(f"  step {i + 1}: {out[-1]:.6g}", flush=True)
    return out


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--configs", default="c3,c5")
    ap.add_argument("--out", default=str(HERE / "loss_curves.json"))
    args = ap.parse_args()
    path = Path(args.out)
    data = json.loads(path.read_text()) if path.exists() else {}
    for name in args.configs.split(","):
        build = BUILDS[name]
        t0 = time.time()
        runs = {}
        print(f"{name}: fused Adam", flush=True)
        runs["cpu_fused"] = curve(build, args.steps, True)
        print(f"{name}: default Adam", flush=True)
        runs["cpu_default"] = curve(build, args.steps, None)
        runs["spread"] = []
        for where in (0, 1, 2):
            print(f"{name}: fused Adam, one weight moved by one ulp ({where})", flush=True)
            runs["spread"].append(curve(build, args.steps, True, where))
        data[name] = {"steps": args.steps, **runs, "seconds": round(time.time() - t0, 1)}
        data["meta"] = {"torch": torch.__version__, "threads": torch.get_num_threads(), "cpu": cpu_model()}
        path.write_text(json.dumps(data, indent=0) + "\n")
        print(f"{name}: done in {time.time() - t0:.0f} s", flush=True)


if __name__ == "__main__":
    main()
