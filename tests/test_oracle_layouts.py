"""Pins the oracle's conv3x3w layout restatement (oracle_pack_strips_range,
oracle_unpack_strips_range).

1. Golden digests of the reference's own conv_pack.cpp (tests/golden/pack_golden.json,
   written by tests/golden/make_pack_golden.py from oracle/_ref) on the shapes of the
   reference's layout test, incl. strips, halo_zero and the 2048/2126 group windows.
2. The reference build itself, where present, on extra seeds and group-range pieces.
3. Layout invariants that a wrong offset would break: unpack of the centre-tap rows of
   a packed input returns the input; group halos duplicate the next group's head.
"""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = json.loads((Path(__file__).parent / "golden" / "pack_golden.json").read_text())["cases"]


def _sha(a):
    import hashlib

    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _inputs(case):
    rng = np.random.default_rng(case["seed"])
    x = oracle.bf16_bits(rng.standard_normal((case["B"], case["C"], case["H"], case["W"])).astype(np.float32))
    raw = rng.integers(0, 65536, (case["groups"] * oracle.GROUP_OUT_ROWS, 128), dtype=np.uint16)
    return x, raw


def _pieces(groups):
    out = [[groups]]
    if groups > 1:
        out.append([groups - groups // 2, groups // 2])
        a = max(1, groups // 5)
        b = max(1, groups // 3)
        if groups - a - b > 0:
            out.append([a, b, groups - a - b])
    if groups <= 8:
        out.append([1] * groups)
    return out


@pytest.mark.parametrize("case", GOLDEN, ids=lambda c: f"B{c['B']}C{c['C']}H{c['H']}W{c['W']}s{int(c['strips'])}")
def test_pack_matches_reference_digest(case):
    x, _ = _inputs(case)
    B, C, H, W = case["B"], case["C"], case["H"], case["W"]
    S, So, chunks, groups = case["S"], case["So"], case["chunks"], case["groups"]
    for hz in ([0, 1] if S > 1 else [0]):
        full = oracle.pack_strips_range(x, B, C, H, W, S, So, hz, chunks, 0, groups)
        assert _sha(full) == case[f"pack_h{hz}"]
        # group-range pieces assemble to the same buffer
        for cuts in _pieces(groups):
            parts, g0 = [], 0
            for n in cuts:
                parts.append(oracle.pack_strips_range(x, B, C, H, W, S, So, hz, chunks, g0, n))
                g0 += n
            assert _sha(np.concatenate(parts)) == case[f"pack_h{hz}"]


@pytest.mark.parametrize("case", GOLDEN, ids=lambda c: f"B{c['B']}C{c['C']}H{c['H']}W{c['W']}s{int(c['strips'])}")
def test_unpack_matches_reference_digest(case):
    _, raw = _inputs(case)
    B, H, W, S, So = case["B"], case["H"], case["W"], case["S"], case["So"]
    cout, cx, cs = case["Cout"], case["c_extra"], case["c_start"]
    nv = min(cout, 128)
    m_total = B * S * (H + 2) * case["wp"]
    out = np.zeros((B, cout + cx, H, W), np.uint16)
    oracle.unpack_strips_range(raw, out, B, H, W, S, So, nv, cout + cx, cs, 0, m_total)
    assert _sha(out) == case["unpack"]
    # arbitrary row ranges (mid-row cuts, one-row pieces) give the same result
    wp = case["wp"]
    cuts = sorted({0, 1, wp + 3, 5 * wp - 1, m_total // 2, m_total - 1, m_total})
    out2 = np.zeros_like(out)
    for a, b in zip(cuts[:-1], cuts[1:]):
        oracle.unpack_strips_range(raw[a:], out2, B, H, W, S, So, nv, cout + cx, cs, a, b)
    assert _sha(out2) == case["unpack"]


@pytest.mark.parametrize("shape", [(1, 1, 1, 1), (2, 65, 3, 40, ), (5, 130, 7, 9), (2, 64, 11, 75),
                                   (3, 17, 2, 100)])
def test_pack_against_reference_build(shape):
    B, C, H, W = shape
    ref = oracle.ref_pack()  # looked up here, not at collection: the GPU box has no build
    if ref is None:
        pytest.skip("reference build (oracle/_ref) absent: the committed digests pin the layouts")
    rng = np.random.default_rng(7 + B + C)
    x = oracle.rng_bf16(rng, (B, C, H, W))
    for strips in (False, True):
        S, So, Wg, wp, m_total, groups = oracle.geometry(B, H, W, strips)
        chunks = -(-C // 64) + (1 if C % 64 == 0 else 0)  # also an extra all-padding chunk
        for hz in ([0, 1] if S > 1 else [0]):
            for cuts in _pieces(groups):
                g0 = 0
                for n in cuts:
                    mine = oracle.pack_strips_range(x, B, C, H, W, S, So, hz, chunks, g0, n)
                    theirs = np.zeros_like(mine)
                    ref.xdna_conv3x3w_pack_input_strips_range_bf16(
                        x.ctypes.data, theirs.ctypes.data, B, C, H, W, S, So, hz, chunks, g0, n)
                    np.testing.assert_array_equal(mine, theirs)
                    g0 += n
        raw = rng.integers(0, 65536, (groups * oracle.GROUP_OUT_ROWS, 128), dtype=np.uint16)
        for nv, ctot, cs in ((min(C, 128), C + 2, 1), (5, 9, 4)):
            mine = np.zeros((B, ctot, H, W), np.uint16)
            theirs = np.zeros_like(mine)
            oracle.unpack_strips_range(raw, mine, B, H, W, S, So, nv, ctot, cs, 0, m_total)
            ref.xdna_conv3x3w_unpack_output_strips_range_bf16(raw.ctypes.data, theirs.ctypes.data, B, H,
                                                              W, S, So, nv, ctot, cs, 0, m_total)
            np.testing.assert_array_equal(mine, theirs)


@pytest.mark.parametrize("B,C,H,W", [(2, 64, 5, 7), (3, 70, 9, 30), (2, 40, 6, 50)])
def test_centre_tap_roundtrip(B, C, H, W):
    """Output row p of the 3x3 window has its centre tap at input row p + wp + 1: copying
    packed rows through that offset and unpacking returns the input (pins pack vs unpack
    offsets, incl. strips)."""
    rng = np.random.default_rng(3)
    x = oracle.rng_bf16(rng, (B, C, H, W))
    S, So, Wg, wp, m_total, groups = oracle.geometry(B, H, W)
    packed = oracle.pack(x, B, C, H, W)  # [groups][chunks][2126][64]
    chunks = packed.shape[1]
    rows = np.zeros((groups * oracle.GROUP_OUT_ROWS + oracle.GROUP_ROWS, chunks * 64), np.uint16)
    for g in range(groups):
        for ch in range(chunks):
            rows[g * 2048:g * 2048 + 2126, ch * 64:(ch + 1) * 64] = packed[g, ch]
    raw = np.zeros((groups * 2048, 128), np.uint16)
    p = np.arange(groups * 2048)
    nv = min(C, 128)
    raw[:, :nv] = rows[p + wp + 1, :nv]
    out = np.zeros((B, C, H, W), np.uint16)
    oracle.unpack_strips_range(raw, out, B, H, W, S, So, nv, C, 0, 0, m_total)
    np.testing.assert_array_equal(out[:, :nv], x[:, :nv])


def test_group_halo_duplicates_next_group():
    rng = np.random.default_rng(5)
    B, C, H, W = 3, 64, 30, 30
    x = oracle.rng_bf16(rng, (B, C, H, W))
    packed = oracle.pack(x, B, C, H, W)
    assert packed.shape[0] >= 2
    for g in range(packed.shape[0] - 1):
        np.testing.assert_array_equal(packed[g, :, 2048:2126], packed[g + 1, :, 0:78])
    # padded channels of a partial chunk stay zero
    x2 = oracle.rng_bf16(rng, (B, 70, H, W))
    p2 = oracle.pack(x2, B, 70, H, W)
    assert not p2[:, 1, :, 6:].any()
