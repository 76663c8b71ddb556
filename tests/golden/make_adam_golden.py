"""Writes tests/golden/adam_golden.npz: inputs and outputs of PyTorch's CPU
``torch._fused_adam_`` / ``torch._fused_adamw_`` on seeded tensors.

That kernel is what the reference runs for fused=True parameter groups on its device
(the boxed CPU fallback, torch_xdna_device.cpp:5124-5260, after
_prefer_fused_optimizer, xdna_train/device.py:408-436).  Produced with the torch in this
container (2.10.0+rocm7.0, CPU).  Each case stores p, g, m, v, max_v before the step
and p, m, v, max_v (and g, for grad_scale) after it.

numel is a multiple of 32 so every element goes through the CPU kernel's vector path
(its scalar tail rounds v without the fused multiply-add).
Run: ``python tests/golden/make_adam_golden.py``.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

N = 1024
CASES = [
    # name, dtype, step, lr, beta1, beta2, eps, wd, amsgrad, maximize, adamw, grad_scale
    ("bf16_s1", torch.bfloat16, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, False, False, False, None),
    ("bf16_s7", torch.bfloat16, 7, 1e-3, 0.9, 0.999, 1e-8, 0.0, False, False, False, None),
    ("bf16_wd", torch.bfloat16, 3, 2e-3, 0.9, 0.999, 1e-8, 0.01, False, False, False, None),
    ("bf16_adamw_ams", torch.bfloat16, 5, 1e-3, 0.9, 0.999, 1e-8, 0.05, True, False, True, None),
    ("bf16_max", torch.bfloat16, 2, 1e-3, 0.8, 0.99, 1e-6, 0.0, False, True, False, None),
    ("bf16_scale", torch.bfloat16, 4, 1e-3, 0.9, 0.999, 1e-8, 0.0, False, False, False, 64.0),
    ("f32_s1", torch.float32, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, False, False, False, None),
    ("f32_s9", torch.float32, 9, 1e-3, 0.9, 0.999, 1e-8, 0.0, False, False, False, None),
    ("f32_adamw_ams", torch.float32, 6, 1e-3, 0.9, 0.999, 1e-8, 0.02, True, False, True, None),
    ("f32_wd", torch.float32, 3, 1e-3, 0.9, 0.999, 1e-8, 0.01, False, False, False, None),
    # beta1 <= 0.5: the first moment's lerp weight 1 - beta1 is >= 0.5, which takes the
    # lerp's other form (computed from the end point)
    ("bf16_b1_03", torch.bfloat16, 3, 1e-3, 0.3, 0.999, 1e-8, 0.0, False, False, False, None),
    ("f32_b1_03", torch.float32, 4, 1e-3, 0.3, 0.99, 1e-8, 0.01, False, False, False, None),
    ("bf16_b1_05", torch.bfloat16, 2, 1e-3, 0.5, 0.999, 1e-8, 0.0, False, False, False, None),
    ("f32_b1_0_ams", torch.float32, 5, 1e-3, 0.0, 0.999, 1e-8, 0.02, True, False, True, None),
]


def main():
    out = {}
    for i, (name, dt, step, lr, b1, b2, eps, wd, ams, mx, adamw, scale) in enumerate(CASES):
        gen = torch.Generator().manual_seed(1234 + i)
        p = (torch.randn(N, generator=gen) * 0.5).to(dt)
        g = (torch.randn(N, generator=gen) * 1e-2).to(dt)
        g[:8] = 0  # zero gradients
        m = (torch.randn(N, generator=gen) * 1e-2).to(dt)
        v = (torch.rand(N, generator=gen) * 1e-4).to(dt)
        mxv = (torch.rand(N, generator=gen) * 1e-4).to(dt)
        if step == 1:
            m.zero_()
            v.zero_()
            mxv.zero_()
        P, G, M, V, MX = (t.clone() for t in (p, g, m, v, mxv))
        st = torch.tensor(float(step))
        fn = torch._fused_adamw_ if adamw else torch._fused_adam_
        kw = {}
        if scale is not None:
            kw["grad_scale"] = torch.tensor(scale)
        fn([P], [G], [M], [V], [MX] if ams else [], [st], lr=lr, beta1=b1, beta2=b2,
           weight_decay=wd, eps=eps, amsgrad=ams, maximize=mx, **kw)
        as_np = (lambda t: t.view(torch.int16).numpy().view(np.uint16)) if dt == torch.bfloat16 \
            else (lambda t: t.numpy())
        for key, t in (("p", p), ("g", g), ("m", m), ("v", v), ("mx", mxv), ("P", P), ("G", G),
                       ("M", M), ("V", V), ("MX", MX)):
            out[f"{name}.{key}"] = as_np(t)
        out[f"{name}.hp"] = np.array([step, lr, b1, b2, eps, wd, float(ams), float(mx),
                                      float(adamw), -1.0 if scale is None else scale])
    path = Path(__file__).with_name("adam_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
