"""Fused training regions on the xdna device: a pattern of eager ops runs as one autograd
node whose forward and backward are fused device passes.

The reference's regions (xdna_train/regions.py:1-425, host kernels in
_native/region_kernels.cpp:51-340) fuse a frozen feature network's perceptual loss on the
CPU.  Here the same contract runs on the GPU:

* the feature network ``Sequential(conv, relu, conv, relu, maxpool, ...)`` is frozen (no
  weight needs a gradient); 3x3 / stride-1 / pad-1 convs followed by a ReLU run as one
  conv whose epilogue applies the ReLU before rounding (no pre-activation tensor, no
  separate ReLU pass);
* tap terms reduce on the device into fixed-order partial sums and one finishing sum, so
  the loss never goes through the host, and the backward reads the incoming loss gradient
  on the device: a step with a region is graph-capturable;
* the backward produces dX only: per layer one pass that applies the ReLU mask, routes a
  max-pool's gradient to its window maxima and adds the tap terms, then the conv's input
  gradient.

Numerics (the reference region's, regions.py:29-32): bf16 storage, fp32 arithmetic in the
fused kernels, one rounding per output.  The conv results equal the eager conv + relu bit
for bit (rounding is monotonic and keeps the sign); loss terms and gradients are within
rounding of the eager path, which rounds the difference, the square and the mean
separately.

Regions (``XDNA_REGIONS=0`` turns them off; anything ineligible runs the eager ops):

* :func:`frozen_feature_mse` / :func:`fuse_perceptual_loss`: the reference's perceptual
  loss, mean over the concatenated tap elements of (features(x) - features(target))^2;
* :func:`frozen_feature_loss`: the same chain with Gram-matrix style terms as well
  (w * mean((F F^T / chw - T)^2) per style tap, the style-transfer loss of the BASELINE
  style configuration), an fp32 loss like the eager ``.float()`` losses it replaces;
* :func:`fuse_norm_activation` / :func:`fuse_norm_activations`: a training BatchNorm2d or
  InstanceNorm2d and the ReLU / LeakyReLU applied to its output as one kernel pair, the
  activation in the norm's output store and its mask in the norm's backward sums.
"""
from __future__ import annotations

import os
import types
import weakref
from dataclasses import dataclass

import torch
import torch.nn as nn
from torch.autograd.function import once_differentiable
from torch.nn.modules import module as _modmod
from torch.nn.utils import parametrize

from . import device as _dev


def enabled() -> bool:
    """Regions are on unless ``XDNA_REGIONS=0`` (the reference's switch)."""
    return os.environ.get("XDNA_REGIONS", "1") != "0"


def _exactly(m: nn.Module, cls) -> bool:
    """m is ``cls`` itself and runs nothing around its forward that a region would skip:
    no instance-level forward, no module or global hooks, no parametrization."""
    if type(m) is not cls or "forward" in m.__dict__:
        return False
    if m._forward_hooks or m._forward_pre_hooks or m._backward_hooks or m._backward_pre_hooks:
        return False
    if _modmod._global_forward_hooks or _modmod._global_forward_pre_hooks:
        return False
    return not parametrize.is_parametrized(m)


def _signature(m: nn.Module):
    """What the chain depends on for one layer (re-checked on every call), or None."""
    if _exactly(m, nn.Conv2d):
        if m.padding_mode != "zeros" or isinstance(m.padding, str):
            return None
        return ("conv", id(m), id(m.weight), id(m.bias), tuple(m.stride), tuple(m.padding), tuple(m.dilation),
                m.groups)
    if _exactly(m, nn.ReLU):
        return ("relu", id(m))
    if _exactly(m, nn.MaxPool2d):
        two = lambda v: v in (2, (2, 2))
        if (two(m.kernel_size) and two(m.stride) and m.padding in (0, (0, 0)) and m.dilation in (1, (1, 1))
                and not m.ceil_mode and not m.return_indices):
            return ("maxpool2", id(m))
    return None


@dataclass
class _Op:
    kind: str                 # "conv" | "relu" | "maxpool2"
    module: nn.Module
    fused_relu: bool = False  # conv whose following ReLU runs in its epilogue


def _conv3x3_s1(m: nn.Conv2d) -> bool:
    return (tuple(m.kernel_size) == (3, 3) and tuple(m.stride) == (1, 1) and tuple(m.padding) == (1, 1)
            and tuple(m.dilation) == (1, 1) and m.groups == 1)


class FrozenFeatureChain:
    """A parsed ``layers[0 .. max(taps)]`` of conv / ReLU / 2x2 max-pool modules with
    frozen weights; ``taps`` are the layer indices whose outputs the loss reads."""

    def __init__(self, layers, taps, sig):
        self.layers = layers
        self.taps = taps
        self.sig = sig
        tapset = set(taps)
        self.ops: list[_Op] = []
        for i, m in enumerate(layers):
            kind = sig[i][0]
            op = _Op(kind, m)
            # conv + ReLU in one launch unless the loss reads the pre-activation
            if (kind == "conv" and i + 1 < len(layers) and sig[i + 1][0] == "relu" and i not in tapset
                    and _conv3x3_s1(m)):
                op.fused_relu = True
            self.ops.append(op)

    @classmethod
    def from_sequential(cls, layers, taps) -> "FrozenFeatureChain | None":
        """The chain of ``layers[0 .. max(taps)]``, or None if a layer is not a plain
        Conv2d / ReLU / MaxPool2d(2, 2), a weight is trainable, or the first layer is not
        a conv (it reads the image)."""
        layers = list(layers)
        taps = tuple(sorted({int(t) for t in taps}))
        if not taps or taps[0] < 0 or taps[-1] >= len(layers):
            return None
        layers = layers[: taps[-1] + 1]
        sig = []
        for m in layers:
            s = _signature(m)
            if s is None:
                return None
            if s[0] == "conv" and (m.weight.requires_grad or (m.bias is not None and m.bias.requires_grad)):
                return None
            sig.append(s)
        if sig[0][0] != "conv":
            return None
        return cls(layers, taps, tuple(sig))

    def current(self) -> bool:
        """The layers still are what the chain was parsed from (strides, hooks, weights)."""
        return tuple(_signature(m) for m in self.layers) == self.sig

    def eligible(self, x: torch.Tensor, target: torch.Tensor | None = None) -> bool:
        if not enabled() or not isinstance(x, torch.Tensor) or x.device.type != "xdna":
            return False
        if x.dtype != torch.bfloat16 or x.dim() != 4:
            return False
        if target is not None and (target.device.type != "xdna" or target.dtype != torch.bfloat16
                                   or target.shape != x.shape or target.requires_grad):
            return False
        if torch.is_grad_enabled() and not x.requires_grad:
            return False  # the region's backward produces dX only
        if not self.current():
            return False
        for op in self.ops:
            if op.kind != "conv":
                continue
            w, b = op.module.weight, op.module.bias
            if w.device.type != "xdna" or w.dtype != torch.bfloat16 or w.requires_grad:
                return False
            if b is not None and (b.device.type != "xdna" or b.dtype != torch.bfloat16 or b.requires_grad):
                return False
        return True


def _run(chain: FrozenFeatureChain, x: torch.Tensor, upto: int):
    """outs[i] = output of layer i for i <= upto (None for a conv whose ReLU is fused)."""
    C = _dev.native()
    outs: list[torch.Tensor | None] = [None] * len(chain.ops)
    cur = x
    i = 0
    while i <= upto:
        op = chain.ops[i]
        m = op.module
        if op.kind == "conv":
            if op.fused_relu and i + 1 <= upto:
                cur = C.region_conv3x3(cur.contiguous(), m.weight, m.bias, 1)
                outs[i + 1] = cur
                i += 2
                continue
            if _conv3x3_s1(m):
                cur = C.region_conv3x3(cur.contiguous(), m.weight, m.bias, 0)
            else:
                cur = torch.nn.functional.conv2d(cur, m.weight, m.bias, m.stride, m.padding, m.dilation, m.groups)
        elif op.kind == "relu":
            cur = torch.relu(cur)
        else:
            cur = C.region_maxpool2(cur.contiguous())
        outs[i] = cur.contiguous()
        cur = outs[i]
        i += 1
    return outs


class _FrozenFeatureLoss(torch.autograd.Function):
    """loss = mse_weight * sum over mse taps of sum (f(x) - f(target))^2 / (their element
    count) + sum over style taps of w * mean((F F^T / chw - T)^2), F the tap as
    [B][C][H*W]."""

    @staticmethod
    def forward(ctx, chain, x, target, mse_taps, style, mse_weight, out_bf16):
        C = _dev.native()
        parts = C.region_loss_parts()
        last = max(list(mse_taps) + list(style.keys()))
        with torch.no_grad():
            outs = _run(chain, x, last)
            t_outs = _run(chain, target, max(mse_taps)) if mse_taps else [None] * len(chain.ops)
            nterms = len(mse_taps) + len(style)
            part = torch.empty(nterms * parts, dtype=torch.float32, device=x.device)
            total = sum(outs[k].numel() for k in mse_taps)
            off = 0
            for k in mse_taps:
                C.region_sqdiff(outs[k], t_outs[k], mse_weight / total, part, off)
                off += parts
            grams = {}
            for k, (T, w) in style.items():
                f = outs[k]
                B, Ch = f.shape[0], f.shape[1]
                F3 = f.view(B, Ch, -1)
                G = C.region_bmm(F3, F3.transpose(1, 2), 1.0)
                Tc = T.to(device=x.device, dtype=torch.float32).reshape(-1, Ch, Ch).contiguous()
                chw = float(f[0].numel())
                C.region_gram_sqdiff(G, Tc, chw, float(w) / G.numel(), part, off)
                off += parts
                grams[k] = (G, Tc, chw, float(w))
            loss_f, loss_h = C.region_loss_finish(part)
        keep = [i for i, t in enumerate(outs) if t is not None]
        tkeep = list(mse_taps)
        gkeep = list(grams.keys())
        ctx.save_for_backward(x, *[outs[i] for i in keep], *[t_outs[i] for i in tkeep],
                              *[grams[k][0] for k in gkeep], *[grams[k][1] for k in gkeep])
        ctx.meta = (chain, keep, tkeep, gkeep, {k: (grams[k][2], grams[k][3]) for k in gkeep}, total, mse_weight,
                    last)
        return loss_h if out_bf16 else loss_f

    @staticmethod
    @once_differentiable
    def backward(ctx, go):
        C = _dev.native()
        chain, keep, tkeep, gkeep, gmeta, total, mse_weight, last = ctx.meta
        saved = ctx.saved_tensors  # raises if a saved tensor was written in place
        x = saved[0]
        n = 1
        outs = [None] * len(chain.ops)
        for i in keep:
            outs[i] = saved[n]
            n += 1
        t_outs = {}
        for k in tkeep:
            t_outs[k] = saved[n]
            n += 1
        Gs = {}
        for k in gkeep:
            Gs[k] = saved[n]
            n += 1
        Ts = {}
        for k in gkeep:
            Ts[k] = saved[n]
            n += 1
        go = go.detach().contiguous()
        mse_scale = 2.0 * mse_weight / total if total else 0.0

        def tap_terms(k):
            ta = tb = extra = None
            if k in t_outs:
                ta, tb = outs[k], t_outs[k]
            if k in Gs:
                f = outs[k]
                chw, w = gmeta[k]
                S = C.region_gram_grad(Gs[k], Ts[k], chw, 2.0 * w / Gs[k].numel(), go)
                F3 = f.view(f.shape[0], f.shape[1], -1)
                extra = C.region_bmm(S, F3, 1.0).view(f.shape)
            return ta, tb, extra

        G = None   # gradient with respect to the output of layer k
        Gp = None  # gradient with respect to a max-pool's output, not yet routed
        for k in range(last, -1, -1):
            op = chain.ops[k]
            if op.kind == "conv" and op.fused_relu:
                pass  # the ReLU above produced the gradient of the pre-activation
            elif op.kind == "maxpool2":
                # gradient of this pool's output: routed from a pool above (whose input
                # this output is) and the tap terms; it is routed to the window maxima of
                # this pool's input by the layer below
                ta, tb, extra = tap_terms(k)
                if Gp is not None or ta is not None or extra is not None:
                    G = C.region_backward(None, G, Gp, outs[k] if Gp is not None else None, extra, ta, tb,
                                          mse_scale, go, list(outs[k].shape))
                Gp, G = G, None
                continue
            else:
                ta, tb, extra = tap_terms(k)
                src = outs[k]
                if op.kind == "relu" or Gp is not None or ta is not None or extra is not None:
                    G = C.region_backward(src if op.kind == "relu" else None, G, Gp, src if Gp is not None else None,
                                          extra, ta, tb, mse_scale, go, list(src.shape))
                    Gp = None
                if op.kind == "relu":
                    continue
            # conv: the input gradient through the backend's conv path (frozen weight: dX only)
            m = op.module
            inp = outs[k - 1] if k > 0 else x
            G = torch.ops.aten.convolution_backward(G, inp, m.weight, None, list(m.stride), list(m.padding),
                                                    list(m.dilation), False, [0, 0], m.groups,
                                                    [True, False, False])[0]
        return None, G, None, None, None, None, None


def frozen_feature_mse(chain: FrozenFeatureChain, x: torch.Tensor, target: torch.Tensor):
    """The reference's perceptual loss (regions.py:346-349): mean over the concatenated
    tap elements of (chain(x)[tap] - chain(target)[tap])^2, a bf16 scalar; the eager ops
    when the region does not apply."""
    if not chain.eligible(x, target):
        return _eager_mse(chain, x, target)
    return _FrozenFeatureLoss.apply(chain, x, target, chain.taps, {}, 1.0, True)


def frozen_feature_loss(chain: FrozenFeatureChain, x: torch.Tensor, target: torch.Tensor | None = None, *,
                        mse_taps=None, style=None, mse_weight: float = 1.0):
    """fp32 loss = mse_weight * (mean over the concatenated ``mse_taps`` elements of
    (chain(x) - chain(target))^2) + sum over ``style`` = {tap: (T, w)} of
    w * mean((F F^T / (C H W) - T)^2), F = chain(x)[tap] as [B][C][H W] and T the target
    Gram matrices ([C][C] or [1 or B][C][C], fp32).  ``mse_taps`` defaults to the chain's
    taps that are not style taps.  Runs the eager ops when the region does not apply."""
    style = dict(style or {})
    if mse_taps is None:
        mse_taps = tuple(t for t in chain.taps if t not in style)
    mse_taps = tuple(sorted(set(int(t) for t in mse_taps)))
    if mse_taps and target is None:
        raise ValueError("frozen_feature_loss: feature taps need a target")
    if not set(mse_taps) | set(style) <= set(chain.taps):
        raise ValueError("frozen_feature_loss: every tap must be one of the chain's taps")
    if not chain.eligible(x, target if mse_taps else None):
        return _eager_loss(chain, x, target, mse_taps, style, mse_weight)
    return _FrozenFeatureLoss.apply(chain, x, target if mse_taps else x.detach(), mse_taps, style, float(mse_weight),
                                    False)


def _eager_features(chain: FrozenFeatureChain, x: torch.Tensor, upto: int):
    outs = []
    cur = x
    for m in chain.layers[: upto + 1]:
        cur = m(cur)
        outs.append(cur)
    return outs


def _eager_mse(chain, x, target):
    fx = _eager_features(chain, x, chain.taps[-1])
    with torch.no_grad():
        ft = _eager_features(chain, target, chain.taps[-1])
    a = torch.cat([fx[k].reshape(-1) for k in chain.taps])
    b = torch.cat([ft[k].reshape(-1) for k in chain.taps])
    return ((a - b) ** 2).mean()


def _eager_loss(chain, x, target, mse_taps, style, mse_weight):
    last = max(list(mse_taps) + list(style.keys()))
    fx = _eager_features(chain, x, last)
    loss = x.new_zeros((), dtype=torch.float32)
    if mse_taps:
        with torch.no_grad():
            ft = _eager_features(chain, target, max(mse_taps))
        a = torch.cat([fx[k].reshape(-1).float() for k in mse_taps])
        b = torch.cat([ft[k].reshape(-1).float() for k in mse_taps])
        loss = loss + mse_weight * torch.nn.functional.mse_loss(a, b)
    for k, (T, w) in style.items():
        f = fx[k]
        F3 = f.reshape(f.shape[0], f.shape[1], -1)
        g = (F3 @ F3.transpose(1, 2)).float() / float(f[0].numel())
        Tc = T.to(device=g.device, dtype=torch.float32).reshape(-1, f.shape[1], f.shape[1])
        loss = loss + float(w) * torch.nn.functional.mse_loss(g, Tc.expand_as(g))
    return loss


# ---------------------------------------------------------------------------------------
# Routing a loss module's perceptual loss through the region (the reference's
# fuse_perceptual_loss, regions.py:351-425)
# ---------------------------------------------------------------------------------------
def _module_chain(loss_module):
    cfg = loss_module.__dict__["_xdna_region_cfg"]
    net = getattr(loss_module, cfg["features_attr"], None)
    feats = getattr(getattr(net, "model", None), "features", None)
    taps = getattr(net, "feature_layers", None)
    if feats is None or taps is None or not len(taps):
        return None
    layers = list(feats)[: max(taps) + 1]
    chain = loss_module.__dict__.get("_xdna_chain")
    if chain is not None and (chain.taps != tuple(sorted({int(t) for t in taps})) or chain.layers != layers
                              or not chain.current()):
        chain = None
    if chain is None:
        chain = FrozenFeatureChain.from_sequential(layers, taps)
        loss_module.__dict__["_xdna_chain"] = chain
    return chain


def _fused_perceptual(self, input, target):
    """Bound to the loss module: everything is read from ``self`` at call time."""
    chain = _module_chain(self)
    if chain is None or not chain.eligible(input, target):
        return type(self).compute_perceptual_loss(self, input, target)
    net = getattr(self, self.__dict__["_xdna_region_cfg"]["features_attr"])
    x, t = input, target
    if getattr(net, "use_norm", False):
        norm = getattr(net, "norm", None)
        mean, std = getattr(norm, "mean", None), getattr(norm, "std", None)
        if mean is None or std is None:
            return type(self).compute_perceptual_loss(self, input, target)
        m = torch.as_tensor(mean, dtype=x.dtype, device=x.device).view(1, -1, 1, 1)
        s = torch.as_tensor(std, dtype=x.dtype, device=x.device).view(1, -1, 1, 1)
        x, t = (x - m) / s, (t - m) / s
    return _FrozenFeatureLoss.apply(chain, x, t, chain.taps, {}, 1.0, True)


def fuse_perceptual_loss(loss_module, features_attr: str = "perceptual_vgg") -> bool:
    """Routes ``loss_module.compute_perceptual_loss`` through the region when the module
    follows the reference's pattern (regions.py:392-425): ``getattr(loss_module,
    features_attr)`` has ``model.features`` (a Sequential), ``feature_layers`` (tap
    indices), optional ``use_norm`` / ``norm`` (mean / std), and the loss is the mean
    squared tap difference.  Every call re-checks eligibility; anything else takes the
    module's own method.  The wrapper is bound to the module, so a deepcopy uses its own
    weights.  Returns True if the region was installed."""
    if not enabled():
        return False
    net = getattr(loss_module, features_attr, None)
    feats = getattr(getattr(net, "model", None), "features", None)
    taps = getattr(net, "feature_layers", None)
    if feats is None or taps is None or not len(taps) or not hasattr(loss_module, "compute_perceptual_loss"):
        return False
    if FrozenFeatureChain.from_sequential(list(feats)[: max(taps) + 1], taps) is None:
        return False
    if getattr(net, "use_norm", False):
        norm = getattr(net, "norm", None)
        if getattr(norm, "mean", None) is None or getattr(norm, "std", None) is None:
            return False
    loss_module.__dict__["_xdna_region_cfg"] = {"features_attr": features_attr}
    loss_module.compute_perceptual_loss = types.MethodType(_fused_perceptual, loss_module)
    return True


# ---------------------------------------------------------------------------------------
# A training norm and the activation applied to its output as one pass each way (the
# reference's fuse_norm_activation, regions.py:426-546), for BatchNorm2d and, beyond the
# reference, InstanceNorm2d
# ---------------------------------------------------------------------------------------
# Smallest input (bytes) that takes the fused op.  On the GPU the fused pair saves a full
# elementwise pass and its launch each way at every size, so every size is fused unless
# this is raised (the reference's knob; its CPU kernels only win above ~4 MB).
_NORM_ACT_MIN_BYTES = int(os.environ.get("XDNA_REGION_NORM_ACT_MIN_BYTES", "0"))


class _NormAct(torch.autograd.Function):
    """y = act(norm(x)) with training statistics on contiguous NCHW bf16, act applied in
    fp32 before the one rounding of y (ReLU: the same bits as the eager norm then relu;
    LeakyReLU: within one rounding of them).  Saved for backward: x, y (the activation's
    mask is read from y), the weight and the fp32 statistics.  Gradients: input, weight and
    bias, each only if requested.  Not double differentiable."""

    @staticmethod
    def forward(ctx, x, weight, bias, running_mean, running_var, momentum, eps, act, slope, instance):
        y, mean, invstd = _dev.native().region_norm_act_fwd(x, weight, bias, running_mean, running_var,
                                                            momentum, eps, act, slope, instance)
        ctx.save_for_backward(x, y, weight, mean, invstd)
        ctx.act, ctx.slope, ctx.instance = act, slope, instance
        return y

    @staticmethod
    @once_differentiable
    def backward(ctx, dy):
        x, y, weight, mean, invstd = ctx.saved_tensors
        need_x, need_w, need_b = ctx.needs_input_grad[0:3]
        dx, dw, db = _dev.native().region_norm_act_bwd(dy, x, y, weight, mean, invstd, ctx.act, ctx.slope,
                                                       ctx.instance, need_x, need_w or need_b)
        return (dx if need_x else None, dw if need_w else None, db if need_b else None,
                None, None, None, None, None, None, None)


def _act_code(act):
    """(code, slope) for the kernels, or None: exact types only (a subclass may override
    forward, which the fused op would skip); a negative slope makes y > 0 no longer the
    input's sign, so it stays eager."""
    if type(act) is nn.ReLU:
        return 1, 0.0
    if type(act) is nn.LeakyReLU and float(act.negative_slope) >= 0.0:
        return 2, float(act.negative_slope)
    return None


def _param_ok(t, x, dtypes):
    return (isinstance(t, torch.Tensor) and t.device == x.device and t.dtype in dtypes and t.is_contiguous()
            and t.dim() == 1 and t.numel() == x.shape[1])


def _norm_act_args(norm, x):
    """(running_mean, running_var, momentum, instance) when the fused op applies, else None."""
    if not enabled() or not norm.affine:
        return None
    # a forward hook may replace the output, which would then be activated twice
    if norm._forward_hooks or _modmod._global_forward_hooks:
        return None
    if not isinstance(x, torch.Tensor) or x.dim() != 4 or x.device.type != "xdna":
        return None
    if x.dtype != torch.bfloat16 or not x.is_contiguous() or x.numel() * 2 < max(_NORM_ACT_MIN_BYTES, 1):
        return None
    floats = (torch.bfloat16, torch.float32)
    w, b = norm.weight, norm.bias
    if not (_param_ok(w, x, floats) and _param_ok(b, x, floats)) or w.dtype != b.dtype:
        return None
    plane = x.shape[2] * x.shape[3]
    if type(norm) is nn.InstanceNorm2d:
        # running statistics (used or updated) stay eager; planes of one element are the
        # eager path's error
        if norm.track_running_stats or plane <= 1 or plane > 65536:
            return None
        return None, None, 0.0, True
    if not norm.training or x.shape[0] * plane <= 1:
        return None
    if not norm.track_running_stats:
        return None, None, 0.0, False
    rm, rv = norm.running_mean, norm.running_var
    if norm.momentum is None or rm is None or rv is None:  # cumulative average: eager
        return None
    if not (_param_ok(rm, x, floats) and _param_ok(rv, x, floats)) or rm.dtype != rv.dtype:
        return None
    return rm, rv, float(norm.momentum), False


def _fused_norm_forward(self, x):
    """Bound to the norm module (a deepcopy rebinds it to the copy).  The paired activation
    and its slope are read from ``self`` at call time."""
    act = self.__dict__.get("_xdna_pair")
    code = _act_code(act) if act is not None else None
    args = _norm_act_args(self, x) if code is not None else None
    if args is None:
        return type(self).forward(self, x)
    rm, rv, momentum, instance = args
    if rm is not None and self.num_batches_tracked is not None:
        self.num_batches_tracked.add_(1)
    y = _NormAct.apply(x, self.weight, self.bias, rm, rv, momentum, float(self.eps), code[0], code[1], instance)
    y._xdna_act_for = weakref.ref(act)
    return y


def _checked_act_forward(self, x):
    """Passes through, once, a tensor that the paired fused norm already activated, and
    activates everything else."""
    ref = getattr(x, "_xdna_act_for", None)
    if ref is not None and ref() is self:
        x._xdna_act_for = None  # consumed: a later call on the same tensor activates it
        return x
    return type(self).forward(self, x)


def fuse_norm_activation(norm: nn.Module, act: nn.Module) -> bool:
    """Declares that ``act`` (nn.ReLU or nn.LeakyReLU) is applied directly to the output of
    ``norm`` (nn.BatchNorm2d or nn.InstanceNorm2d) and runs the pair as one fused op each
    way, like the reference's fuse_norm_activation (regions.py:521-546).

    Both modules keep their parameters, buffers and state_dict keys; only their forwards
    are replaced, by methods bound to the modules, so a deepcopy of a model with the pair
    gives a working pair (copy the two together: the pairing is stored on the norm).  When
    the fused op applies (affine; BatchNorm2d in training mode with tracked statistics and
    a float momentum, or none tracked; InstanceNorm2d without running statistics; bf16
    contiguous NCHW on xdna), ``norm(x)`` returns the activated tensor and the next call of
    ``act`` on exactly that tensor passes it through once; anything else runs both modules
    unchanged.  The activation's slope is read on every call.

    The pairing is the caller's statement about the model's dataflow: if the activation is
    not applied to the norm's output directly (an add or a branch in between), do not
    declare the pair.  Returns True if installed (or already installed with ``act``)."""
    if not enabled() or type(norm) not in (nn.BatchNorm2d, nn.InstanceNorm2d):
        return False
    if type(act) not in (nn.ReLU, nn.LeakyReLU):
        return False
    if norm.__dict__.get("_xdna_pair") is not None:
        return norm.__dict__["_xdna_pair"] is act
    object.__setattr__(norm, "_xdna_pair", act)  # a plain attribute, not a submodule
    norm.forward = types.MethodType(_fused_norm_forward, norm)
    if not isinstance(act.forward, types.MethodType) or act.forward.__func__ is not _checked_act_forward:
        act.forward = types.MethodType(_checked_act_forward, act)
    return True


def fuse_norm_activations(model: nn.Module) -> int:
    """Pairs, in every nn.Sequential of ``model`` (or subclass that keeps its forward), each
    BatchNorm2d / InstanceNorm2d that is immediately followed by a ReLU / LeakyReLU (such a
    container feeds each module's output straight to the next, so the dataflow statement
    holds).  Returns the pairs installed."""
    n = 0
    for m in model.modules():
        if not isinstance(m, nn.Sequential) or type(m).forward is not nn.Sequential.forward:
            continue
        if "forward" in m.__dict__ or m._forward_hooks:
            continue
        mods = list(m)
        for a, b in zip(mods, mods[1:]):
            if type(a) in (nn.BatchNorm2d, nn.InstanceNorm2d) and type(b) in (nn.ReLU, nn.LeakyReLU):
                n += bool(fuse_norm_activation(a, b))
    return n
