"""CPU oracle of the MI355X hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
may import this package, and only as the checker (or the timed CPU baseline).  The
product path (``pytorch-xdna2_amd/``) never imports, links or runs it.

Contents:

* ``liboracle.so`` (``oracle.c``): plain-C restatements of the conv3x3w layouts
  (pack / unpack, with strips, halo_zero and group ranges), the BFP16 weight codec
  (forward and dX forms), the BFP16 emulation of the NPU's conv arithmetic (block
  quantization, bf16 running sum per chunk and tap), the direct 3x3 convolution forward / input-gradient /
  weight-gradient / bias-gradient in double precision, and the fused Adam step.
* numpy helpers: bf16 rounding, the GEMM reference (float64 products of bf16 values),
  and the layout geometry.
* ``ref_pack()``: the reference's own ``conv_pack.cpp`` compiled in place into
  ``oracle/_ref/conv_pack.so`` (only where ``/root/reference`` exists); a second
  checker for the layouts.

Pinning (what proves each function right) is recorded in the tests that use it:
``tests/test_oracle_layouts.py`` (reference build + committed golden digests + layout
invariants), ``tests/test_oracle_conv.py`` (brute force, closed forms, linearity,
torch CPU fp32 convolution), ``tests/test_oracle_bfp16.py`` (reference build + committed
golden digests + closed forms), ``tests/test_oracle_adam.py`` (golden vectors from
torch's CPU ``_fused_adam_`` + known-answer steps), ``tests/test_oracle_gemm.py``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
GROUP_OUT_ROWS = 2048
GROUP_ROWS = 2126
KSTEP = 64
RAW_N = 128

_lib = None
_ref = None

P = ctypes.c_void_p
I = ctypes.c_int
L = ctypes.c_int64
D = ctypes.c_double


def lib():
    """liboracle.so, built with make if missing."""
    global _lib
    if _lib is None:
        so = HERE / "liboracle.so"
        if not so.exists():
            subprocess.check_call(["make", "-s", "-C", str(HERE), "liboracle.so"])
        _lib = ctypes.CDLL(str(so))
        _lib.oracle_pack_strips_range.argtypes = [P, P, I, I, I, I, I, I, I, I, I, I]
        _lib.oracle_unpack_strips_range.argtypes = [P, P, I, I, I, I, I, I, I, I, L, L]
        _lib.oracle_conv3x3_fwd.argtypes = [P, P, P, P, I, I, I, I, I]
        _lib.oracle_conv3x3_dgrad.argtypes = [P, P, P, I, I, I, I, I]
        _lib.oracle_conv3x3_wgrad.argtypes = [P, P, P, P, I, I, I, I, I]
        _lib.oracle_adam.argtypes = [P, P, P, P, P, L, I, D, D, D, D, D, D, I, I, I, D, I]
        _lib.oracle_strip_geometry.argtypes = [I, ctypes.POINTER(I), ctypes.POINTER(I)]
        _lib.oracle_pack_weights_bfp16.argtypes = [P, P, I, I, I, I, I, I]
        _lib.oracle_bfp16_quantize8.argtypes = [P, P, L]
        _lib.oracle_conv3x3_bfp16_emul.argtypes = [P, P, P, P, I, I, I, I, I]
    return _lib


def ref_pack():
    """The reference's conv_pack.cpp built in oracle/_ref (None when unavailable)."""
    global _ref
    if _ref is None:
        so = HERE / "_ref" / "conv_pack.so"
        if not so.exists():
            return None
        _ref = ctypes.CDLL(str(so))
        _ref.xdna_conv3x3w_pack_input_strips_range_bf16.argtypes = [P, P, I, I, I, I, I, I, I, I, I, I]
        _ref.xdna_conv3x3w_unpack_output_strips_range_bf16.argtypes = [P, P, I, I, I, I, I, I, I, I, I]
        _ref.xdna_conv3x3w_pack_input_bf16.argtypes = [P, P, I, I, I, I, I]
        _ref.xdna_conv3x3w_unpack_output_bf16.argtypes = [P, P, I, I, I, I, I, I]
        _ref.xdna_conv_set_threads.argtypes = [I]
        _ref.xdna_conv3x3w_pack_weights_bfp16.argtypes = [P, P, I, I, I, I]
        _ref.xdna_conv3x3w_pack_weights_dx_bfp16.argtypes = [P, P, I, I, I, I]
    return _ref


# ---------------------------------------------------------------------------
# bf16
# ---------------------------------------------------------------------------

def bf16_bits(x) -> np.ndarray:
    """float -> bf16 bit patterns, round to nearest even (NaN -> 0x7FC0)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u + (np.uint32(0x7FFF) + ((u >> 16) & 1))) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    if nan.any():
        r = np.where(nan, np.uint16(0x7FC0), r)
    return r


def bf16_value(bits) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_ulp(x) -> np.ndarray:
    """Spacing of bf16 numbers at |x| (the ulp of the bf16 value nearest x)."""
    a = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, np.finfo(np.float32).tiny)))
    return np.exp2(e - 7)


def rng_bf16(rng, shape, scale=1.0) -> np.ndarray:
    return bf16_bits(rng.standard_normal(shape).astype(np.float32) * np.float32(scale))


# ---------------------------------------------------------------------------
# layouts
# ---------------------------------------------------------------------------

def strip_geometry(W: int) -> tuple[int, int]:
    S, So = I(), I()
    lib().oracle_strip_geometry(W, ctypes.byref(S), ctypes.byref(So))
    return S.value, So.value


def geometry(B: int, H: int, W: int, strips: bool = True):
    """(S, So, Wg, wp, m_total, groups) of the padded-grid layout."""
    S, So = strip_geometry(W) if strips else (1, W)
    Wg = W if S == 1 else So + 2
    wp = Wg + 2
    m_total = B * S * (H + 2) * wp
    groups = -(-m_total // GROUP_OUT_ROWS)
    return S, So, Wg, wp, m_total, groups


def pack_strips_range(src_bits: np.ndarray, B, C, H, W, S, So, halo_zero, chunks, g0, ng,
                      out: np.ndarray | None = None) -> np.ndarray:
    src = np.ascontiguousarray(src_bits, dtype=np.uint16)
    if out is None:
        out = np.zeros((ng, chunks, GROUP_ROWS, KSTEP), np.uint16)
    lib().oracle_pack_strips_range(src.ctypes.data, out.ctypes.data, B, C, H, W, S, So,
                                   int(halo_zero), chunks, g0, ng)
    return out


def pack(src_bits, B, C, H, W, halo_zero=False, strips=True):
    S, So, Wg, wp, m_total, groups = geometry(B, H, W, strips)
    chunks = -(-C // KSTEP)
    return pack_strips_range(src_bits, B, C, H, W, S, So, halo_zero, chunks, 0, groups)


def unpack_strips_range(c_bits, out, B, H, W, S, So, cout_valid, C_total, c_start, p0, p1):
    c = np.ascontiguousarray(c_bits, dtype=np.uint16)
    assert out.dtype == np.uint16 and out.flags.c_contiguous
    lib().oracle_unpack_strips_range(c.ctypes.data, out.ctypes.data, B, H, W, S, So, cout_valid,
                                     C_total, c_start, p0, p1)
    return out


# ---------------------------------------------------------------------------
# convolution (double accumulation of bf16 operands)
# ---------------------------------------------------------------------------

def conv3x3_fwd(x_bits, w_bits, bias_bits=None):
    B, Cin, H, W = x_bits.shape
    Cout = w_bits.shape[0]
    x = np.ascontiguousarray(x_bits, np.uint16)
    w = np.ascontiguousarray(w_bits, np.uint16)
    b = None if bias_bits is None else np.ascontiguousarray(bias_bits, np.uint16)
    y = np.empty((B, Cout, H, W), np.float64)
    lib().oracle_conv3x3_fwd(x.ctypes.data, w.ctypes.data, None if b is None else b.ctypes.data,
                             y.ctypes.data, B, Cin, Cout, H, W)
    return y


def conv3x3_dgrad(dy_bits, w_bits):
    B, Cout, H, W = dy_bits.shape
    Cin = w_bits.shape[1]
    dy = np.ascontiguousarray(dy_bits, np.uint16)
    w = np.ascontiguousarray(w_bits, np.uint16)
    dx = np.empty((B, Cin, H, W), np.float64)
    lib().oracle_conv3x3_dgrad(dy.ctypes.data, w.ctypes.data, dx.ctypes.data, B, Cin, Cout, H, W)
    return dx


def conv3x3_wgrad(x_bits, dy_bits):
    B, Cin, H, W = x_bits.shape
    Cout = dy_bits.shape[1]
    x = np.ascontiguousarray(x_bits, np.uint16)
    dy = np.ascontiguousarray(dy_bits, np.uint16)
    gw = np.empty((Cout, Cin, 3, 3), np.float64)
    gb = np.empty((Cout,), np.float64)
    lib().oracle_conv3x3_wgrad(x.ctypes.data, dy.ctypes.data, gw.ctypes.data, gb.ctypes.data,
                               B, Cin, Cout, H, W)
    return gw, gb


# ---------------------------------------------------------------------------
# GEMM and Adam
# ---------------------------------------------------------------------------

def gemm(a_bits, b_bits, bias_bits=None, alpha=1.0, beta=1.0):
    """alpha * A.B (+ beta * bias) in float64 from bf16 operands ([..., M, K] x [..., K, N])."""
    a = bf16_value(a_bits).astype(np.float64)
    b = bf16_value(b_bits).astype(np.float64)
    c = alpha * np.matmul(a, b)
    if bias_bits is not None and beta != 0:
        c = c + beta * bf16_value(bias_bits).astype(np.float64)
    return c


def adam_(p, g, m, v, mx, step, lr=1e-3, beta1=0.9, beta2=0.999, weight_decay=0.0, eps=1e-8,
          amsgrad=False, maximize=False, adamw=False, grad_scale=None):
    """In-place fused Adam on numpy arrays (uint16 bf16 bits or float32)."""
    dtype = 1 if p.dtype == np.uint16 else 0
    for t in (p, g, m, v) + ((mx,) if amsgrad else ()):
        assert t.flags.c_contiguous and t.dtype == p.dtype
    lib().oracle_adam(p.ctypes.data, g.ctypes.data, m.ctypes.data, v.ctypes.data,
                      mx.ctypes.data if amsgrad else None, p.size, dtype, float(step), lr, beta1,
                      beta2, weight_decay, eps, int(amsgrad), int(maximize), int(adamw),
                      0.0 if grad_scale is None else float(grad_scale), int(grad_scale is not None))


# ---------------------------------------------------------------------------
# BFP16 weight codec
# ---------------------------------------------------------------------------

BFP16_BYTES_PER_CHUNK = 9 * 8 * 8 * 2 * 8 * 9   # one 128-channel block: 82,944 per chunk


def pack_weights_bfp16(w_bits: np.ndarray, chunks: int, n_block: int) -> np.ndarray:
    """OIHW bf16 bits -> bfp16ebs8 bytes of output channels [128 n_block, +128)."""
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    cout, cin = w.shape[:2]
    out = np.zeros(chunks * BFP16_BYTES_PER_CHUNK, np.uint8)
    lib().oracle_pack_weights_bfp16(w.ctypes.data, out.ctypes.data, cout, cin, cin, chunks, n_block, 0)
    return out


def pack_weights_dx_bfp16(w_bits: np.ndarray, chunks: int, n_block: int) -> np.ndarray:
    """The dX conv's bfp16 weights, read from the forward weight [Cout_fwd][Cin_fwd][3][3]."""
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    cout_fwd, cin_fwd = w.shape[:2]
    out = np.zeros(chunks * BFP16_BYTES_PER_CHUNK, np.uint8)
    lib().oracle_pack_weights_bfp16(w.ctypes.data, out.ctypes.data, cin_fwd, cout_fwd, cin_fwd, chunks,
                                    n_block, 1)
    return out


def bfp16_decode(blocks: np.ndarray) -> np.ndarray:
    """9-byte blocks -> float64 values (int8 mantissa * 2^(e - 133))."""
    b = np.asarray(blocks, np.uint8).reshape(-1, 9)
    e = b[:, :1].astype(np.int64)
    m = b[:, 1:].view(np.int8).astype(np.float64)
    return np.ldexp(m, e - 133).reshape(-1)


# ---------------------------------------------------------------------------
# BFP16 emulation of the reference NPU's conv arithmetic (oracle.c: quantization as the
# codec's blocks decode; chunk-major, tap-inner bf16 running sum; bias after)
# ---------------------------------------------------------------------------

def bfp16_quantize8(bits: np.ndarray) -> np.ndarray:
    """bf16 bits (size a multiple of 8) -> the BFP16 values of each aligned run of 8, as bf16 bits."""
    src = np.ascontiguousarray(bits, dtype=np.uint16)
    assert src.size % 8 == 0
    out = np.empty_like(src)
    lib().oracle_bfp16_quantize8(src.ctypes.data, out.ctypes.data, src.size // 8)
    return out


def conv3x3_bfp16_emul(x_bits, w_bits, bias_bits=None) -> np.ndarray:
    """The NPU-arithmetic forward conv (3x3, stride 1, pad 1) -> bf16 bits [B, Cout, H, W]."""
    B, Cin, H, W = x_bits.shape
    Cout = w_bits.shape[0]
    x = np.ascontiguousarray(x_bits, np.uint16)
    w = np.ascontiguousarray(w_bits, np.uint16)
    b = None if bias_bits is None else np.ascontiguousarray(bias_bits, np.uint16)
    y = np.empty((B, Cout, H, W), np.uint16)
    lib().oracle_conv3x3_bfp16_emul(x.ctypes.data, w.ctypes.data, None if b is None else b.ctypes.data,
                                    y.ctypes.data, B, Cin, Cout, H, W)
    return y


def conv3x3_dgrad_bfp16_emul(dy_bits, w_bits) -> np.ndarray:
    """The NPU-arithmetic input gradient: the emulated forward conv of dY with the flipped,
    swapped weights w'[ci][co][t] = w[co][ci][8 - t] (conv_pack.cpp:470-473)."""
    wd = np.ascontiguousarray(np.asarray(w_bits, np.uint16)[:, :, ::-1, ::-1].transpose(1, 0, 2, 3))
    return conv3x3_bfp16_emul(dy_bits, wd)


# ---------------------------------------------------------------------------
# General 2-D convolution (any kernel, stride, padding; dilation 1, groups 1), float64
# of bf16 operands.  The reference runs these on PyTorch's CPU kernels
# (torch_xdna_device.cpp:4524-4606, 4608-4885); restated here as sums over the kernel
# taps of strided slices of the zero-padded input.
# ---------------------------------------------------------------------------

def _f64(bits):
    return bf16_value(bits).astype(np.float64)


def conv2d_out_size(H, W, KH, KW, sh, sw, ph, pw):
    return (H + 2 * ph - KH) // sh + 1, (W + 2 * pw - KW) // sw + 1


def conv2d_fwd(x_bits, w_bits, bias_bits=None, stride=(1, 1), padding=(0, 0)):
    x, w = _f64(x_bits), _f64(w_bits)
    B, Cin, H, W = x.shape
    Cout, _, KH, KW = w.shape
    (sh, sw), (ph, pw) = stride, padding
    Ho, Wo = conv2d_out_size(H, W, KH, KW, sh, sw, ph, pw)
    xp = np.zeros((B, Cin, H + 2 * ph, W + 2 * pw))
    xp[:, :, ph:ph + H, pw:pw + W] = x
    y = np.zeros((B, Cout, Ho, Wo))
    for ky in range(KH):
        for kx in range(KW):
            sl = xp[:, :, ky:ky + sh * (Ho - 1) + 1:sh, kx:kx + sw * (Wo - 1) + 1:sw]
            y += np.einsum("bchw,oc->bohw", sl, w[:, :, ky, kx], optimize=True)
    if bias_bits is not None:
        y += _f64(bias_bits)[None, :, None, None]
    return y


def conv2d_dgrad(dy_bits, w_bits, in_hw, stride=(1, 1), padding=(0, 0)):
    dy, w = _f64(dy_bits), _f64(w_bits)
    B, Cout, Ho, Wo = dy.shape
    _, Cin, KH, KW = w.shape
    (sh, sw), (ph, pw) = stride, padding
    H, W = in_hw
    dxp = np.zeros((B, Cin, max(H + 2 * ph, sh * (Ho - 1) + KH), max(W + 2 * pw, sw * (Wo - 1) + KW)))
    for ky in range(KH):
        for kx in range(KW):
            dxp[:, :, ky:ky + sh * (Ho - 1) + 1:sh, kx:kx + sw * (Wo - 1) + 1:sw] += np.einsum(
                "bohw,oc->bchw", dy, w[:, :, ky, kx], optimize=True)
    return dxp[:, :, ph:ph + H, pw:pw + W]


def conv2d_wgrad(x_bits, dy_bits, kernel, stride=(1, 1), padding=(0, 0)):
    x, dy = _f64(x_bits), _f64(dy_bits)
    B, Cin, H, W = x.shape
    _, Cout, Ho, Wo = dy.shape
    KH, KW = kernel
    (sh, sw), (ph, pw) = stride, padding
    xp = np.zeros((B, Cin, H + 2 * ph, W + 2 * pw))
    xp[:, :, ph:ph + H, pw:pw + W] = x
    gw = np.zeros((Cout, Cin, KH, KW))
    for ky in range(KH):
        for kx in range(KW):
            sl = xp[:, :, ky:ky + sh * (Ho - 1) + 1:sh, kx:kx + sw * (Wo - 1) + 1:sw]
            gw[:, :, ky, kx] = np.einsum("bohw,bchw->oc", dy, sl, optimize=True)
    return gw, dy.sum(axis=(0, 2, 3))
