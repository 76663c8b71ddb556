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
  (w * mean((F F^T / chw - T)^2) per style tap, the loss of a style-transfer training
  step), an fp32 loss like the eager ``.float()`` losses it replaces;
* :func:`fuse_norm_activation` / :func:`fuse_norm_activations`: a training BatchNorm2d or
  InstanceNorm2d and the ReLU / LeakyReLU applied to its output as one kernel pair, the
  activation in the norm's output store and its mask in the norm's backward sums.
"""
from __future__ import annotations

import os
import weakref

import torch
import torch.nn as nn
from torch.autograd.function import once_differentiable
from torch.nn.modules import module as _modmod
from torch.nn.utils import parametrize

from . import device as _dev


def enabled() -> bool:
    """Regions are on unless ``XDNA_REGIONS=0`` (the reference's switch)."""
    return os.environ.get("XDNA_REGIONS", "1") != "0"


def _call_extras(m: nn.Module) -> tuple:
    """What calling ``m`` runs besides ``type(m).forward``, whose arithmetic is all a
    region reproduces: an instance-level forward, module or global hooks, a
    parametrization.  Empty for a module that is called plainly."""
    found = []
    if "forward" in vars(m):
        found.append("instance forward")
    for attr in ("_forward_pre_hooks", "_forward_hooks", "_backward_pre_hooks", "_backward_hooks"):
        if len(getattr(m, attr)):
            found.append(attr.lstrip("_"))
    if len(_modmod._global_forward_pre_hooks) or len(_modmod._global_forward_hooks):
        found.append("global forward hooks")
    if parametrize.is_parametrized(m):
        found.append("parametrization")
    return tuple(found)


def _conv_state(m: nn.Conv2d):
    if m.padding_mode != "zeros" or isinstance(m.padding, str):
        return None
    return (m.weight, m.bias, tuple(m.stride), tuple(m.padding), tuple(m.dilation), m.groups)


def _pool2_state(m: nn.MaxPool2d):
    def pair(v, want):
        return v == want or v == (want, want)
    shape_ok = pair(m.kernel_size, 2) and pair(m.stride, 2) and pair(m.padding, 0) and pair(m.dilation, 1)
    return () if shape_ok and not m.ceil_mode and not m.return_indices else None


# exact module type -> (kind, state function); a state is what the region's result depends
# on beyond the kind, or None when the module's configuration is not supported
_LAYER_KINDS = {
    nn.Conv2d: ("conv", _conv_state),
    nn.ReLU: ("relu", lambda m: ()),
    nn.MaxPool2d: ("maxpool2", _pool2_state),
}


def _describe(m: nn.Module):
    """(kind, state) of a layer the region can run, else None.  Exact types only: a
    subclass may compute something else in its forward."""
    entry = _LAYER_KINDS.get(type(m))
    if entry is None or _call_extras(m):
        return None
    state = entry[1](m)
    return None if state is None else (entry[0], state)


def _same_description(a, b) -> bool:
    """Descriptions compared with tensors by identity (a replaced weight is a new layer)."""
    if a is None or b is None or a[0] != b[0] or len(a[1]) != len(b[1]):
        return False
    for u, v in zip(a[1], b[1]):
        if isinstance(u, torch.Tensor) or isinstance(v, torch.Tensor):
            if u is not v:
                return False
        elif u != v:
            return False
    return True


def _conv3x3_s1(m: nn.Conv2d) -> bool:
    return (tuple(m.kernel_size) == (3, 3) and tuple(m.stride) == (1, 1) and tuple(m.padding) == (1, 1)
            and tuple(m.dilation) == (1, 1) and m.groups == 1)


class FrozenFeatureChain:
    """A parsed ``layers[0 .. max(taps)]`` of conv / ReLU / 2x2 max-pool modules with
    frozen weights; ``taps`` are the layer indices whose outputs the loss reads.

    ``kinds[i]`` is layer i's kind ("conv", "relu" or "maxpool2"); ``fused_relu[i]`` is
    True for a 3x3 stride-1 conv that applies the following ReLU in its epilogue (not
    done when the loss reads the conv's own output)."""

    def __init__(self, layers, taps, descriptions):
        self.layers = layers
        self.taps = taps
        self._descriptions = descriptions
        self.kinds = tuple(d[0] for d in descriptions)
        read = set(taps)
        self.fused_relu = tuple(
            k == "conv" and i + 1 < len(layers) and self.kinds[i + 1] == "relu" and i not in read
            and _conv3x3_s1(layers[i])
            for i, k in enumerate(self.kinds))

    @classmethod
    def from_sequential(cls, layers, taps) -> "FrozenFeatureChain | None":
        """The chain of ``layers[0 .. max(taps)]``, or None when some layer is not a plain
        Conv2d / ReLU / MaxPool2d(2, 2), a conv parameter is trainable, or the first layer
        is not a conv (the region's first pass reads the image through a conv)."""
        taps = tuple(sorted({int(t) for t in taps}))
        layers = list(layers)
        if not taps or taps[0] < 0 or taps[-1] >= len(layers):
            return None
        layers = layers[: taps[-1] + 1]
        descriptions = tuple(_describe(m) for m in layers)
        if any(d is None for d in descriptions) or descriptions[0][0] != "conv":
            return None
        for m, d in zip(layers, descriptions):
            if d[0] == "conv" and any(p.requires_grad for p in m.parameters(recurse=False)):
                return None
        return cls(layers, taps, descriptions)

    def current(self) -> bool:
        """The layers are still what the chain was parsed from (types, strides, hooks, the
        weight and bias objects)."""
        return all(_same_description(_describe(m), d) for m, d in zip(self.layers, self._descriptions))

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
        for m, kind in zip(self.layers, self.kinds):
            if kind != "conv":
                continue
            w, b = m.weight, m.bias
            if w.device.type != "xdna" or w.dtype != torch.bfloat16 or w.requires_grad:
                return False
            if b is not None and (b.device.type != "xdna" or b.dtype != torch.bfloat16 or b.requires_grad):
                return False
        return True


def _run(chain: FrozenFeatureChain, x: torch.Tensor, upto: int):
    """outs[i] = output of layer i for i <= upto (None for a conv whose ReLU is fused)."""
    C = _dev.native()
    outs: list[torch.Tensor | None] = [None] * len(chain.layers)
    cur = x
    i = 0
    while i <= upto:
        m, kind = chain.layers[i], chain.kinds[i]
        if kind == "conv":
            if chain.fused_relu[i] and i + 1 <= upto:
                cur = C.region_conv3x3(cur.contiguous(), m.weight, m.bias, 1)
                outs[i + 1] = cur
                i += 2
                continue
            if _conv3x3_s1(m):
                cur = C.region_conv3x3(cur.contiguous(), m.weight, m.bias, 0)
            else:
                cur = torch.nn.functional.conv2d(cur, m.weight, m.bias, m.stride, m.padding, m.dilation, m.groups)
        elif kind == "relu":
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
            t_outs = _run(chain, target, max(mse_taps)) if mse_taps else [None] * len(chain.layers)
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
        outs = [None] * len(chain.layers)
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
            kind = chain.kinds[k]
            if kind == "conv" and chain.fused_relu[k]:
                pass  # the ReLU above produced the gradient of the pre-activation
            elif kind == "maxpool2":
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
                if kind == "relu" or Gp is not None or ta is not None or extra is not None:
                    G = C.region_backward(src if kind == "relu" else None, G, Gp, src if Gp is not None else None,
                                          extra, ta, tb, mse_scale, go, list(src.shape))
                    Gp = None
                if kind == "relu":
                    continue
            # conv: the input gradient through the backend's conv path (frozen weight: dX only)
            m = chain.layers[k]
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
# A loss module's perceptual loss through the region (the interface of the reference's
# fuse_perceptual_loss, regions.py:392-425)
# ---------------------------------------------------------------------------------------
def _perceptual_layers(net):
    """(layers, taps) of a feature network in the loss-module pattern: ``net.model.features``
    (a Sequential) and ``net.feature_layers`` (tap indices); None otherwise."""
    feats = getattr(getattr(net, "model", None), "features", None)
    taps = getattr(net, "feature_layers", None)
    if feats is None or taps is None or len(taps) == 0:
        return None
    taps = tuple(sorted({int(t) for t in taps}))
    return list(feats)[: taps[-1] + 1], taps


def _input_normalizer(net):
    """``(mean, std)`` the network applies to its inputs first (``use_norm`` with a ``norm``
    holding both), ``()`` when it applies none, None when it names a norm the region
    cannot reproduce."""
    if not getattr(net, "use_norm", False):
        return ()
    norm = getattr(net, "norm", None)
    mean, std = getattr(norm, "mean", None), getattr(norm, "std", None)
    return None if mean is None or std is None else (mean, std)


class _PerceptualRoute:
    """What ``loss_module.compute_perceptual_loss`` becomes once routed: a callable that
    holds its module (``owner``) and the name of the feature network's attribute, and
    decides on every call between the region and the class's own method.

    It is an instance attribute of the module, so ``copy.deepcopy`` of the module copies it
    with ``owner`` pointing at the copy (deepcopy's memo), and the copy runs on its own
    weights.  The parsed chain is kept with the layer identities it was parsed from and
    rebuilt when the module's feature layers, taps or their state change."""

    def __init__(self, owner, features_attr: str):
        self.owner = owner
        self.features_attr = features_attr
        self._parsed = None  # (layer ids, taps, chain or None)

    def chain(self):
        found = _perceptual_layers(getattr(self.owner, self.features_attr, None))
        if found is None:
            return None
        layers, taps = found
        ids = tuple(id(m) for m in layers)
        parsed = self._parsed
        fresh = parsed is not None and parsed[:2] == (ids, taps) and parsed[2] is not None and parsed[2].current()
        if not fresh:  # a layer that did not parse may have become eligible since
            parsed = self._parsed = (ids, taps, FrozenFeatureChain.from_sequential(layers, taps))
        return parsed[2]

    def __call__(self, input, target):
        chain = self.chain()
        scale = _input_normalizer(getattr(self.owner, self.features_attr, None))
        if chain is None or scale is None or not chain.eligible(input, target):
            return type(self.owner).compute_perceptual_loss(self.owner, input, target)
        if scale:
            shape = (1, -1, 1, 1)
            mean = torch.as_tensor(scale[0], dtype=input.dtype, device=input.device).view(shape)
            std = torch.as_tensor(scale[1], dtype=input.dtype, device=input.device).view(shape)
            input, target = (input - mean) / std, (target - mean) / std
        return _FrozenFeatureLoss.apply(chain, input, target, chain.taps, {}, 1.0, True)


def fuse_perceptual_loss(loss_module, features_attr: str = "perceptual_vgg") -> bool:
    """Routes ``loss_module.compute_perceptual_loss(input, target)`` through the region.

    The module must follow the loss-module pattern: ``getattr(loss_module, features_attr)``
    has ``model.features`` (a Sequential), ``feature_layers`` (tap indices) and optionally
    ``use_norm`` with a ``norm`` holding ``mean`` / ``std``; its loss is the mean squared
    difference of the concatenated taps.  Returns False, installing nothing, when the
    pattern or the chain does not fit now.  Once installed, every call checks again and
    falls back to the class's own ``compute_perceptual_loss`` for anything the region does
    not take (trainable or replaced feature layers, other dtypes or devices)."""
    if not enabled() or not hasattr(loss_module, "compute_perceptual_loss"):
        return False
    net = getattr(loss_module, features_attr, None)
    found = _perceptual_layers(net)
    if found is None or _input_normalizer(net) is None:
        return False
    if FrozenFeatureChain.from_sequential(*found) is None:
        return False
    vars(loss_module)["compute_perceptual_loss"] = _PerceptualRoute(loss_module, features_attr)
    return True


def perceptual_route(loss_module):
    """The installed route of ``fuse_perceptual_loss`` (its ``chain()`` is the parsed
    region), or None."""
    route = vars(loss_module).get("compute_perceptual_loss")
    return route if isinstance(route, _PerceptualRoute) else None


# ---------------------------------------------------------------------------------------
# A training norm and the activation applied to its output, one kernel each way (the
# interface of the reference's fuse_norm_activation, regions.py:521-546, for BatchNorm2d
# and, beyond the reference, InstanceNorm2d)
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


# Activations the fused kernels apply: exact type -> kernel code.  A subclass may override
# forward, which the fused op would skip.
_ACT_KERNEL_CODES = {nn.ReLU: 1, nn.LeakyReLU: 2}
_NORM_TYPES = (nn.BatchNorm2d, nn.InstanceNorm2d)


def _act_kernel_args(act):
    """(code, slope) for the kernels, or None.  A negative LeakyReLU slope stays eager: the
    backward reads the activation's mask from the output's sign, which then flips."""
    code = _ACT_KERNEL_CODES.get(type(act))
    slope = float(getattr(act, "negative_slope", 0.0)) if code == 2 else 0.0
    return None if code is None or slope < 0.0 else (code, slope)


def _vector_like(t, x, dtypes) -> bool:
    """t is a contiguous 1-D per-channel tensor of x on x's device."""
    return (isinstance(t, torch.Tensor) and t.device == x.device and t.dtype in dtypes and t.is_contiguous()
            and t.dim() == 1 and t.numel() == x.shape[1])


def _norm_plan(norm, x):
    """How the fused kernels run ``norm`` on ``x``: (running_mean, running_var, momentum,
    per_image), or None when the module's own forward must run (eval mode, running
    statistics the kernels do not keep, unsupported tensors)."""
    if not enabled() or not norm.affine or len(norm._forward_hooks) or len(_modmod._global_forward_hooks):
        return None  # a forward hook may replace the output, which would then be activated twice
    if not isinstance(x, torch.Tensor) or x.device.type != "xdna" or x.dtype != torch.bfloat16:
        return None
    if x.dim() != 4 or not x.is_contiguous() or 2 * x.numel() < max(_NORM_ACT_MIN_BYTES, 1):
        return None
    params = (torch.bfloat16, torch.float32)
    if not (_vector_like(norm.weight, x, params) and _vector_like(norm.bias, x, params)
            and norm.weight.dtype == norm.bias.dtype):
        return None
    plane = x.shape[2] * x.shape[3]
    if type(norm) is nn.InstanceNorm2d:
        # statistics per (image, channel) plane; running statistics stay eager, and so do
        # one-element planes (the eager path's error)
        ok = not norm.track_running_stats and 1 < plane <= 65536
        return (None, None, 0.0, True) if ok else None
    if not norm.training or x.shape[0] * plane <= 1:
        return None
    if not norm.track_running_stats:
        return None, None, 0.0, False
    rm, rv = norm.running_mean, norm.running_var
    if norm.momentum is None or not (_vector_like(rm, x, params) and _vector_like(rv, x, params)):
        return None  # a cumulative average (momentum None) stays eager
    return (rm, rv, float(norm.momentum), False) if rm.dtype == rv.dtype else None


class _ActivationGuard:
    """``act.forward`` of a paired activation.  It keeps weak references to the tensors that
    fused norms returned already activated for it; a call on one of them returns it
    unchanged and forgets it (one pass-through per fused output), and any other call runs
    the activation's class forward.  One activation may serve several norms."""

    def __init__(self, act):
        self.act = act
        self._ready = []

    def expect(self, y):
        self._ready = [r for r in self._ready if r() is not None]
        self._ready.append(weakref.ref(y))

    def awaits(self, y) -> bool:
        return any(r() is y for r in self._ready)

    def __call__(self, x):
        for i, r in enumerate(self._ready):
            if r() is x:
                del self._ready[i]
                return x
        return type(self.act).forward(self.act, x)

    def __getstate__(self):  # a copy starts with nothing pending
        return {"act": self.act, "_ready": []}


class _FusedNorm:
    """``norm.forward`` of a paired norm: one fused kernel pair when ``_norm_plan`` accepts the
    call and the paired activation is still guarded, else the norm's class forward (the
    activation then runs its own).  Holds both modules, so a deepcopy of a model holding
    both gets a pair of the copies."""

    def __init__(self, norm, act):
        self.norm = norm
        self.act = act

    def __call__(self, x):
        norm, act = self.norm, self.act
        guard = vars(act).get("forward")
        kernel = _act_kernel_args(act) if isinstance(guard, _ActivationGuard) else None
        plan = _norm_plan(norm, x) if kernel is not None else None
        if plan is None:
            return type(norm).forward(norm, x)
        running_mean, running_var, momentum, per_image = plan
        if running_mean is not None and norm.num_batches_tracked is not None:
            norm.num_batches_tracked.add_(1)
        y = _NormAct.apply(x, norm.weight, norm.bias, running_mean, running_var, momentum, float(norm.eps),
                           kernel[0], kernel[1], per_image)
        guard.expect(y)
        return y


def paired_activation(norm: nn.Module):
    """The activation ``norm`` is paired with by ``fuse_norm_activation``, or None."""
    fused = vars(norm).get("forward")
    return fused.act if isinstance(fused, _FusedNorm) else None


def awaits_activation(y: torch.Tensor, act: nn.Module) -> bool:
    """True if ``y`` is a fused norm's output that ``act`` will pass through unchanged."""
    guard = vars(act).get("forward")
    return isinstance(guard, _ActivationGuard) and guard.awaits(y)


def fuse_norm_activation(norm: nn.Module, act: nn.Module) -> bool:
    """Declares that ``act`` (nn.ReLU or nn.LeakyReLU) is applied directly to the output of
    ``norm`` (nn.BatchNorm2d or nn.InstanceNorm2d), so the pair runs as one fused kernel
    each way.

    Both modules keep their parameters, buffers and state_dict keys: the pairing lives in
    callable instance attributes that replace the two forwards (``norm.forward`` holds the
    pair, ``act.forward`` guards the activation), and a deepcopy of a model holding both
    modules gives a working pair of the copies.  When the fused op applies (affine;
    BatchNorm2d in training mode with tracked statistics and a float momentum, or none
    tracked; InstanceNorm2d without running statistics; bf16 contiguous NCHW on xdna),
    ``norm(x)`` returns the activated tensor and the next call of ``act`` on exactly that
    tensor returns it unchanged; anything else runs both modules unchanged.  The
    activation's slope is read on every call.

    The caller states the dataflow: an activation that is not applied to the norm's output
    directly (an add or a branch in between) must not be declared.  Returns True if the
    pair is installed now or was already installed with ``act``."""
    if not enabled() or type(norm) not in _NORM_TYPES or type(act) not in _ACT_KERNEL_CODES:
        return False
    current = paired_activation(norm)
    if current is not None:
        return current is act
    if not isinstance(vars(act).get("forward"), _ActivationGuard):
        vars(act)["forward"] = _ActivationGuard(act)
    vars(norm)["forward"] = _FusedNorm(norm, act)
    return True


def unfuse_norm_activation(norm: nn.Module) -> None:
    """Removes the pairing of ``norm`` (its activation keeps its guard, which passes through
    nothing once no norm expects it)."""
    if isinstance(vars(norm).get("forward"), _FusedNorm):
        del vars(norm)["forward"]


def fuse_norm_activations(model: nn.Module) -> int:
    """Pairs, in every nn.Sequential of ``model`` whose forward is Sequential's own, each
    BatchNorm2d / InstanceNorm2d directly followed by a ReLU / LeakyReLU: such a container
    feeds each module's output straight to the next, so the pairing's dataflow statement
    holds.  Returns the number of pairs installed."""
    n = 0
    for seq in model.modules():
        if not isinstance(seq, nn.Sequential) or type(seq).forward is not nn.Sequential.forward:
            continue
        if "forward" in vars(seq) or len(seq._forward_hooks):
            continue
        children = list(seq)
        for first, second in zip(children, children[1:]):
            if type(first) in _NORM_TYPES and type(second) in _ACT_KERNEL_CODES:
                n += bool(fuse_norm_activation(first, second))
    return n
