"""HIP fused Adam vs PyTorch's CPU torch._fused_adam_ (golden vectors) and the oracle.

Bar: bit-exact (BASELINE asks for 1 bf16 ulp).  Covers bf16 and fp32, weight decay,
AdamW + amsgrad, maximize, grad_scale (incl. the written-back gradient), found_inf,
more tensors than one launch takes, unaligned views (scalar path), ragged and empty
tensors.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from gpu_util import host, stream
from xdna_train import hip_abi

pytestmark = pytest.mark.gpu

G = np.load(Path(__file__).parent / "golden" / "adam_golden.npz")
NAMES = sorted({k.split(".")[0] for k in G.files})


def _dev(a):
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).cuda()
    return torch.from_numpy(a.copy()).cuda()


def _call(hip, ps, gs, ms, vs, mxs, steps, dtype, hp, grad_scale=None, found_inf=None):
    n = len(ps)
    arr = lambda ts: hip_abi.ptr_array([t.data_ptr() if t is not None else None for t in ts])
    rc = hip.xdna_fused_adam(
        n, arr(ps), arr(gs), arr(ms), arr(vs), arr(mxs) if mxs else None, arr(steps),
        hip_abi.int64_array([t.numel() for t in ps]), dtype, hp["lr"], hp["beta1"], hp["beta2"],
        hp["wd"], hp["eps"], int(hp["amsgrad"]), int(hp["maximize"]), int(hp["adamw"]),
        None if grad_scale is None else grad_scale.data_ptr(),
        None if found_inf is None else found_inf.data_ptr(), stream())
    assert rc == 0, hip_abi.last_error()


@pytest.mark.parametrize("name", NAMES)
def test_golden(hip, name):
    step, lr, b1, b2, eps, wd, ams, mx, adamw, scale = G[f"{name}.hp"]
    hp = dict(lr=lr, beta1=b1, beta2=b2, wd=wd, eps=eps, amsgrad=bool(ams), maximize=bool(mx),
              adamw=bool(adamw))
    p, g, m, v, mxv = (_dev(G[f"{name}.{k}"]) for k in ("p", "g", "m", "v", "mx"))
    st = torch.tensor([float(step)], device="cuda")
    dtype = 1 if G[f"{name}.p"].dtype == np.uint16 else 0
    gs = torch.tensor([float(scale)], device="cuda") if scale > 0 else None
    _call(hip, [p], [g], [m], [v], [mxv] if ams else None, [st], dtype, hp, grad_scale=gs)
    np.testing.assert_array_equal(host(p), G[f"{name}.P"])
    np.testing.assert_array_equal(host(m), G[f"{name}.M"])
    np.testing.assert_array_equal(host(v), G[f"{name}.V"])
    if ams:
        np.testing.assert_array_equal(host(mxv), G[f"{name}.MX"])
    if scale > 0:
        np.testing.assert_array_equal(host(g), G[f"{name}.G"])


@pytest.mark.parametrize("dtype", [0, 1])
def test_many_ragged_unaligned_tensors(hip, dtype):
    rng = np.random.default_rng(dtype)
    sizes = [0, 1, 7, 8, 9, 1000, 8191, 8192, 65537] + [int(s) for s in rng.integers(1, 5000, 30)]
    hp = dict(lr=1e-3, beta1=0.9, beta2=0.999, wd=0.01, eps=1e-8, amsgrad=False, maximize=False,
              adamw=False)
    host_arrays, dev_t = [], []
    for i, n in enumerate(sizes):
        arrs = []
        for scale in (0.5, 1e-2, 1e-2, 1e-4):
            a = (rng.standard_normal(n + 1) * scale).astype(np.float32)
            if scale == 1e-4:
                a = np.abs(a)
            arrs.append(oracle.bf16_bits(a) if dtype == 1 else a)
        host_arrays.append(arrs)
        ts = [_dev(a) for a in arrs]
        # odd tensors: a view starting one element in (not 16-byte aligned)
        off = i % 2
        dev_t.append([t[off:off + n] for t in ts])
    steps = [torch.tensor([3.0], device="cuda") for _ in sizes]
    _call(hip, [d[0] for d in dev_t], [d[1] for d in dev_t], [d[2] for d in dev_t], [d[3] for d in dev_t],
          None, steps, dtype, hp)
    for i, n in enumerate(sizes):
        off = i % 2
        p, g, m, v = (np.ascontiguousarray(a[off:off + n]) for a in host_arrays[i])
        oracle.adam_(p, g, m, v, v, 3, lr=1e-3, weight_decay=0.01)
        np.testing.assert_array_equal(host(dev_t[i][0]), p)
        np.testing.assert_array_equal(host(dev_t[i][2]), m)
        np.testing.assert_array_equal(host(dev_t[i][3]), v)


def test_found_inf_skips_the_step(hip):
    p = torch.ones(100, device="cuda")
    g = torch.ones(100, device="cuda")
    m = torch.zeros(100, device="cuda")
    v = torch.zeros(100, device="cuda")
    st = torch.tensor([1.0], device="cuda")
    hp = dict(lr=1e-3, beta1=0.9, beta2=0.999, wd=0.0, eps=1e-8, amsgrad=False, maximize=False, adamw=False)
    _call(hip, [p], [g], [m], [v], None, [st], 0, hp, found_inf=torch.tensor([1.0], device="cuda"))
    assert torch.equal(p, torch.ones_like(p)) and torch.equal(m, torch.zeros_like(m))
    _call(hip, [p], [g], [m], [v], None, [st], 0, hp, found_inf=torch.tensor([0.0], device="cuda"))
    assert not torch.equal(p, torch.ones_like(p))
