"""The recorded CPU loss curves (tests/golden/loss_curves.json, written by
tests/golden/make_loss_curves.py) are what their recipe computes: 200 steps per run of
configs 3 and 5, every run descending, the spread runs apart from the plain run (one
weight moved by one bf16 ulp), and the first steps of config 3's fused-Adam run recomputed
here with the same seeded build (CPU bf16, threads may differ: within 1e-3 relative)."""
import json
from pathlib import Path

import pytest
import torch

import bench

PATH = Path(__file__).resolve().parent / "golden" / "loss_curves.json"


@pytest.fixture(scope="module")
def curves():
    if not PATH.exists():
        pytest.skip("loss_curves.json not recorded")
    return json.loads(PATH.read_text())


@pytest.mark.parametrize("name", ["c3", "c5"])
def test_fixture_structure(curves, name):
    d = curves[name]
    assert d["steps"] == 200
    runs = [d["cpu_fused"], d["cpu_default"], *d["spread"]]
    assert len(d["spread"]) == 3
    for r in runs:
        assert len(r) == 200 and all(v == v and v > 0 for v in r)
        assert sum(r[-10:]) < sum(r[:10])  # descends
    assert any(a != b for a, b in zip(d["spread"][0], d["cpu_fused"]))
    assert {"torch", "threads", "cpu"} <= set(curves["meta"])


def test_c3_first_steps_recomputed(curves):
    step, _ = bench.build_mlp(torch, torch.device("cpu"), fused=True)
    got = [float(step().detach()) for _ in range(3)]
    for g, r in zip(got, curves["c3"]["cpu_fused"][:3]):
        assert abs(g - r) <= 1e-3 * abs(r), (got, curves["c3"]["cpu_fused"][:3])
