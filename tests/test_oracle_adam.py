"""Pins the oracle's fused Adam (oracle_adam).

* Golden vectors of PyTorch's CPU torch._fused_adam_/_fused_adamw_ (the reference's
  fused-optimizer path), tests/golden/adam_golden.npz from make_adam_golden.py:
  bf16 and fp32, weight decay, AdamW + amsgrad, maximize, grad_scale.  Bit-exact.
* Known answers: at step 1 with m = v = 0, |dp| = lr * |g| / (|g| + eps) (about lr for
  |g| >> eps); a zero gradient leaves p unchanged.
"""
from pathlib import Path

import numpy as np
import pytest

import oracle

G = np.load(Path(__file__).parent / "golden" / "adam_golden.npz")
NAMES = sorted({k.split(".")[0] for k in G.files})


@pytest.mark.parametrize("name", NAMES)
def test_matches_torch_cpu_fused_adam(name):
    step, lr, b1, b2, eps, wd, ams, mx, adamw, scale = G[f"{name}.hp"]
    p, g, m, v, mxv = (G[f"{name}.{k}"].copy() for k in ("p", "g", "m", "v", "mx"))
    oracle.adam_(p, g, m, v, mxv, step, lr=lr, beta1=b1, beta2=b2, weight_decay=wd, eps=eps,
                 amsgrad=bool(ams), maximize=bool(mx), adamw=bool(adamw),
                 grad_scale=None if scale < 0 else scale)
    np.testing.assert_array_equal(p, G[f"{name}.P"])
    np.testing.assert_array_equal(m, G[f"{name}.M"])
    np.testing.assert_array_equal(v, G[f"{name}.V"])
    if ams:
        np.testing.assert_array_equal(mxv, G[f"{name}.MX"])
    if scale > 0:
        np.testing.assert_array_equal(g, G[f"{name}.G"])


def test_step_one_known_answer():
    rng = np.random.default_rng(0)
    n = 4096
    p = rng.standard_normal(n).astype(np.float32)
    g = (rng.standard_normal(n) * 1e-2).astype(np.float32)
    g[:16] = 0.0
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    p0 = p.copy()
    lr, eps = 1e-3, 1e-8
    oracle.adam_(p, g, m, v, v, 1, lr=lr, eps=eps)
    dp = p - p0
    np.testing.assert_array_equal(dp[:16], 0.0)
    exp = -lr * g / (np.abs(g) + eps)
    np.testing.assert_allclose(dp[16:], exp[16:], rtol=2e-3, atol=1e-7)
    np.testing.assert_allclose(m, 0.1 * g, rtol=1e-6)
    np.testing.assert_allclose(v, 0.001 * g * g, rtol=1e-5)
