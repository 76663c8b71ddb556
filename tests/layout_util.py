"""Host-side construction of the packed row layouts of the 3x3 conv operands (a test
helper): the reference's conv3x3w layout (layout 0) and the tight strip layout (layout 1).

Rows of 64 channels; virtual image vb = b * S + s has (H + 2) grid rows of wp positions;
data column j (source column s * So - 1 + j for strips, j for one strip) of image row y
sits at grid row (vb * (H + 2) + y + 1) * wp + lead + j.  Groups of 2048 output rows
hold 2126 rows (the last 78 repeat the next group's first 78).  Output row p is centred
on grid row p + wp + 1; output column c of a strip is output row position c + first.
"""
from __future__ import annotations

import numpy as np

GROUP_OUT, GROUP_ROWS, KSTEP = 2048, 2126, 64


def strip_params(W: int, layout: int):
    """(S, So, Wg, wp, lead, first) of a width-W image in `layout`."""
    if W <= 36:
        S, So, Wg, wp, lead = 1, W, W, W + 2, 1
    elif layout == 1:
        S = -(-W // 36)
        So = -(-W // S)
        S, So, Wg, wp, lead = S, So, So + 2, So + 2, 0
    else:
        S = -(-W // 34)
        So = -(-W // S)
        S, So, Wg, wp, lead = S, So, So + 2, So + 4, 1
    first = (1 if S > 1 else 0) + lead - 1
    return S, So, Wg, wp, lead, first


def geometry(B: int, H: int, W: int, layout: int):
    S, So, Wg, wp, lead, first = strip_params(W, layout)
    m_total = B * S * (H + 2) * wp
    return S, So, Wg, wp, lead, first, m_total, -(-m_total // GROUP_OUT)


def flat_rows(x: np.ndarray, layout: int) -> np.ndarray:
    """[groups * 2048 + 78][chunks * 64] grid rows of NCHW x (any dtype; zeros elsewhere)."""
    B, C, H, W = x.shape
    S, So, Wg, wp, lead, first, m_total, groups = geometry(B, H, W, layout)
    chunks = -(-C // KSTEP)
    flat = np.zeros((groups * GROUP_OUT + GROUP_ROWS - GROUP_OUT, chunks * KSTEP), x.dtype)
    for s in range(S):
        for j in range(Wg):
            col = (0 if S == 1 else s * So - 1) + j
            if col < 0 or col >= W:
                continue
            rows = ((np.arange(B)[:, None] * S + s) * (H + 2) + np.arange(H)[None, :] + 1) * wp + lead + j
            flat[rows.reshape(-1), :C] = x[:, :, :, col].transpose(0, 2, 1).reshape(B * H, C)
    return flat


def pack_expected(x_bits: np.ndarray, layout: int) -> np.ndarray:
    """[groups][chunks][2126][64] uint16: the packed input in `layout`."""
    flat = flat_rows(np.ascontiguousarray(x_bits, dtype=np.uint16), layout)
    groups = (flat.shape[0] - (GROUP_ROWS - GROUP_OUT)) // GROUP_OUT
    chunks = flat.shape[1] // KSTEP
    out = np.empty((groups, chunks, GROUP_ROWS, KSTEP), np.uint16)
    for g in range(groups):
        out[g] = flat[g * GROUP_OUT:g * GROUP_OUT + GROUP_ROWS].reshape(GROUP_ROWS, chunks, KSTEP).transpose(1, 0, 2)
    return out


def conv_by_rows(x: np.ndarray, w: np.ndarray, layout: int) -> np.ndarray:
    """float64 3x3 / pad-1 conv computed the way the rows kernels do: output row p sums
    grid rows p + dy * wp + dx against tap (dy, dx), then output rows map back to pixels."""
    B, C, H, W = x.shape
    Cout = w.shape[0]
    S, So, Wg, wp, lead, first, m_total, groups = geometry(B, H, W, layout)
    flat = flat_rows(x.astype(np.float64), layout)
    out_rows = np.zeros((m_total, Cout))
    for dy in range(3):
        for dx in range(3):
            off = dy * wp + dx
            out_rows += flat[off:off + m_total, :C] @ w[:, :, dy, dx].T.astype(np.float64)
    y = np.zeros((B, Cout, H, W))
    img = (H + 2) * wp
    for b in range(B):
        for s in range(S):
            cols = W if S == 1 else min(So, W - s * So)
            for yy in range(H):
                p0 = (b * S + s) * img + yy * wp + first
                x0 = 0 if S == 1 else s * So
                y[b, :, yy, x0:x0 + cols] = out_rows[p0:p0 + cols].T
    return y
