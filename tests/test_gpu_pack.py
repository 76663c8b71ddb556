"""HIP pack/unpack vs the oracle and the reference digests: bit-exact.

Cases: every golden case (the reference layout test's shapes), group-range pieces,
reuse of a buffer across halo modes without re-zeroing (the reference's "zero-fill once
per shape" contract, conv_pack.cpp:625-631), the non-strip entry points, and ragged
channel counts.
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from gpu_util import dev, dev_zeros, host, ptr, stream

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "pack_golden.json").read_text())["cases"]


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _inputs(case):
    rng = np.random.default_rng(case["seed"])
    x = oracle.bf16_bits(rng.standard_normal((case["B"], case["C"], case["H"], case["W"])).astype(np.float32))
    raw = rng.integers(0, 65536, (case["groups"] * oracle.GROUP_OUT_ROWS, 128), dtype=np.uint16)
    return x, raw


@pytest.mark.parametrize("case", GOLDEN, ids=lambda c: f"B{c['B']}C{c['C']}H{c['H']}W{c['W']}s{int(c['strips'])}")
def test_pack_unpack_golden(hip, case):
    x, raw = _inputs(case)
    B, C, H, W = case["B"], case["C"], case["H"], case["W"]
    S, So, chunks, groups = case["S"], case["So"], case["chunks"], case["groups"]
    print(f"pack case B{B} C{C} H{H} W{W} S{S}", flush=True)
    dx = dev(x)
    buf = dev_zeros((groups, chunks, oracle.GROUP_ROWS, 64))
    # other halo mode first: the real one must overwrite it without re-zeroing
    modes = [1, 0, 1] if S > 1 else [0]
    for hz in modes:
        rc = hip.xdna_conv3x3w_pack_input_strips_range_bf16(ptr(dx), ptr(buf), B, C, H, W, S, So, hz,
                                                            chunks, 0, groups, stream())
        assert rc == 0
        got = host(buf)
        assert _sha(got) == case[f"pack_h{hz}"], f"halo_zero={hz}"
    # group-range pieces into separate buffers
    for hz in ([0, 1] if S > 1 else [0]):
        cuts = [groups - groups // 2, groups // 2] if groups > 1 else [1]
        parts, g0 = [], 0
        for n in cuts:
            if n == 0:
                continue
            pb = dev_zeros((n, chunks, oracle.GROUP_ROWS, 64))
            assert hip.xdna_conv3x3w_pack_input_strips_range_bf16(ptr(dx), ptr(pb), B, C, H, W, S, So,
                                                                  hz, chunks, g0, n, stream()) == 0
            parts.append(host(pb))
            g0 += n
        assert _sha(np.concatenate(parts)) == case[f"pack_h{hz}"]
    # unpack, whole and in row ranges
    cout, cx, cs = case["Cout"], case["c_extra"], case["c_start"]
    nv = min(cout, 128)
    m_total = B * S * (H + 2) * case["wp"]
    draw = dev(raw)
    out = dev_zeros((B, cout + cx, H, W))
    assert hip.xdna_conv3x3w_unpack_output_strips_range_bf16(ptr(draw), ptr(out), B, H, W, S, So, nv,
                                                             cout + cx, cs, 0, m_total, stream()) == 0
    assert _sha(host(out)) == case["unpack"]
    out2 = dev_zeros((B, cout + cx, H, W))
    wp = case["wp"]
    cuts = sorted({0, 1, wp + 3, 5 * wp - 1, m_total // 2, m_total - 1, m_total})
    for a, b in zip(cuts[:-1], cuts[1:]):
        sub = draw[a:]
        assert hip.xdna_conv3x3w_unpack_output_strips_range_bf16(ptr(sub), ptr(out2), B, H, W, S, So,
                                                                 nv, cout + cx, cs, a, b, stream()) == 0
    assert _sha(host(out2)) == case["unpack"]


@pytest.mark.parametrize("B,C,H,W", [(2, 65, 3, 40), (5, 130, 7, 9), (1, 1, 1, 1), (3, 17, 2, 100)])
def test_plain_entry_points_match_oracle(hip, B, C, H, W):
    """xdna_conv3x3w_pack_input_bf16 / _range and unpack_output_bf16 / _range (no strips,
    any width), against the oracle with S = 1."""
    print(f"plain case B{B} C{C} H{H} W{W}", flush=True)
    rng = np.random.default_rng(B + C + W)
    x = oracle.rng_bf16(rng, (B, C, H, W))
    S, So, Wg, wp, m_total, groups = oracle.geometry(B, H, W, strips=False)
    chunks = -(-C // 64)
    exp = oracle.pack_strips_range(x, B, C, H, W, 1, W, 0, chunks, 0, groups)
    dx = dev(x)
    buf = dev_zeros(exp.shape)
    assert hip.xdna_conv3x3w_pack_input_bf16(ptr(dx), ptr(buf), B, C, H, W, chunks, stream()) == 0
    np.testing.assert_array_equal(host(buf), exp)
    if groups > 1:
        n = groups // 2
        pb = dev_zeros((n,) + exp.shape[1:])
        assert hip.xdna_conv3x3w_pack_input_range_bf16(ptr(dx), ptr(pb), B, C, H, W, chunks, 1, n,
                                                       stream()) == 0
        np.testing.assert_array_equal(host(pb), oracle.pack_strips_range(x, B, C, H, W, 1, W, 0, chunks, 1, n))
    raw = rng.integers(0, 65536, (groups * 2048, 128), dtype=np.uint16)
    nv = min(C, 128)
    exp_out = np.zeros((B, C + 1, H, W), np.uint16)
    oracle.unpack_strips_range(raw, exp_out, B, H, W, 1, W, nv, C + 1, 1, 0, m_total)
    out = dev_zeros((B, C + 1, H, W))
    assert hip.xdna_conv3x3w_unpack_output_bf16(ptr(dev(raw)), ptr(out), B, H, W, nv, C + 1, 1,
                                                stream()) == 0
    np.testing.assert_array_equal(host(out), exp_out)
    out2 = dev_zeros((B, C + 1, H, W))
    draw = dev(raw)
    half = m_total // 2
    for a, b in ((0, half), (half, m_total)):
        assert hip.xdna_conv3x3w_unpack_output_range_bf16(ptr(draw[a:]), ptr(out2), B, H, W, nv, C + 1,
                                                          1, a, b, stream()) == 0
    np.testing.assert_array_equal(host(out2), exp_out)


def test_unaligned_buffers_take_the_scalar_path(hip):
    """dst / c not 16-byte aligned (views at an odd element offset)."""
    rng = np.random.default_rng(9)
    B, C, H, W = 2, 64, 6, 6
    x = oracle.rng_bf16(rng, (B, C, H, W))
    S, So, Wg, wp, m_total, groups = oracle.geometry(B, H, W)
    exp = oracle.pack_strips_range(x, B, C, H, W, S, So, 0, 1, 0, groups)
    big = dev_zeros((exp.size + 1,))
    assert hip.xdna_conv3x3w_pack_input_strips_range_bf16(ptr(dev(x)), ptr(big[1:]), B, C, H, W, S, So,
                                                          0, 1, 0, groups, stream()) == 0
    np.testing.assert_array_equal(host(big)[1:].reshape(exp.shape), exp)
    raw = rng.integers(0, 65536, (groups * 2048 * 128 + 1,), dtype=np.uint16)
    exp_out = np.zeros((B, C, H, W), np.uint16)
    oracle.unpack_strips_range(raw[1:], exp_out, B, H, W, S, So, 64, C, 0, 0, m_total)
    out = dev_zeros((B, C, H, W))
    assert hip.xdna_conv3x3w_unpack_output_strips_range_bf16(ptr(dev(raw)[1:]), ptr(out), B, H, W, S, So,
                                                             64, C, 0, 0, m_total, stream()) == 0
    np.testing.assert_array_equal(host(out), exp_out)
