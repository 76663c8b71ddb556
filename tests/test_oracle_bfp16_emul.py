"""Pins the oracle's BFP16-emulation restatement (oracle_bfp16_quantize8,
oracle_conv3x3_bfp16_emul): the reference NPU's conv arithmetic, restated on the CPU by
the reference's benchmarks/bfp16_training_gate.py:33-57.

1. Quantization against the BFP16 codec, which the reference's own conv_pack.cpp pins
   (test_oracle_bfp16.py): the values the codec's blocks decode to, for every block of a
   weight, special values included (NaN aside: the codec writes 0, the emulation keeps
   NaN, as the reference's conv gives NaN outputs for NaN operands).
2. Quantization closed forms: zero runs, runs that are already BFP16 values, ties to
   even, the 127 clamp, values below the block's step.
3. The conv with operands and sums exactly representable (small integers, sums within
   bf16's exact integers): the emulation equals the exact conv, so tap offsets, borders,
   the chunk split and the bias add are pinned independently of rounding.
4. The reference gate's own formulation, restated with torch CPU ops (float quantization
   floor(log2(max|v|)), F.unfold im2col, 64-column matmuls with the running sum rounded
   to bf16, K order (tap, channel)), which for 64 channels visits the (chunk, tap) steps in
   the NPU's order: forward and input gradient agree bit for bit.
5. Size of the effect: the emulation's error against the exact conv is larger than one
   bf16 rounding and of the order the reference documents (~1 %, docs/performance.md:62-64).
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("cin,cout,kind", [(64, 128, "recipe"), (130, 40, "recipe"), (64, 72, "special")])
def test_quantization_is_the_codec_decoded(cin, cout, kind):
    from test_oracle_bfp16 import bfp16_weights  # the reference test's weight recipe

    w = np.ascontiguousarray(bfp16_weights(cin, cout, kind, 5))
    chunks = -(-cin // 64)
    for nb in range(-(-cout // 128)):
        blocks = oracle.pack_weights_bfp16(w, chunks, nb)
        with np.errstate(over="ignore"):
            dec = oracle.bfp16_decode(blocks).astype(np.float32)  # +-inf where the decode overflows
        # codec block order [kb][n/16][k/8][2][8 n][8 k] -> [n][kb][k]
        dec = dec.reshape(chunks * 9, 8, 8, 2, 8, 8).transpose(1, 3, 4, 0, 2, 5).reshape(128, chunks * 9, 64)
        want = (dec.view(np.uint32) >> 16).astype(np.uint16)
        # the same runs as the emulation quantizes them: w[n][chunk*64 + c][tap], zero padded
        runs = np.zeros((128, chunks, 9, 64), np.uint16)
        n_hi = min(cout, 128 * nb + 128)
        wn = w[128 * nb:n_hi].reshape(n_hi - 128 * nb, cin, 9)
        for ch in range(chunks):
            c1 = min(cin, ch * 64 + 64)
            runs[:n_hi - 128 * nb, ch, :, :c1 - ch * 64] = wn[:, ch * 64:c1, :].transpose(0, 2, 1)
        got = oracle.bfp16_quantize8(runs).reshape(128, chunks * 9, 64)
        isnan = np.isnan(oracle.bf16_value(runs.reshape(128, chunks * 9, 64)))
        np.testing.assert_array_equal(got[~isnan], want[~isnan])
        assert np.all(got[isnan] == 0x7FC0)


def _q(vals):
    b = oracle.bf16_bits(np.asarray(vals, np.float32))
    return oracle.bf16_value(oracle.bfp16_quantize8(b)).astype(np.float64)


def test_quantization_closed_forms():
    assert np.all(_q(np.zeros(8)) == 0)
    ints = np.array([64, -3, 5, 127, 0, 1, -100, 7], np.float64)
    for s in (2.0 ** -20, 2.0 ** -5, 1.0, 2.0 ** 40):  # already BFP16 values: unchanged
        np.testing.assert_array_equal(_q(ints * s), ints * s)
    # largest value 1.0: step 2^-6; 2^-10 is below half a step, 2^-7 a tie (to even: 0),
    # 3 * 2^-7 a tie (to even: 2 steps), 0.75 * 2^-6 rounds to 1 step
    np.testing.assert_array_equal(_q([1.0, 2.0 ** -10, 2.0 ** -7, 3 * 2.0 ** -7, 0.75 * 2.0 ** -6, -1.0, 0, 0]),
                                  [1.0, 0.0, 0.0, 2 * 2.0 ** -6, 2.0 ** -6, -1.0, 0, 0])
    # 1.9921875 (bf16's largest significand) is 127.5 steps: the clamp keeps 127 (-128 below)
    np.testing.assert_array_equal(_q([1.9921875, -1.9921875, 0, 0, 0, 0, 0, 0]),
                                  [127 * 2.0 ** -6, -128 * 2.0 ** -6, 0, 0, 0, 0, 0, 0])
    q = _q([np.nan, 1.0, 0, 0, 0, 0, 0, 0])
    assert np.isnan(q[0])


def _small_int_case(B, Cin, Cout, H, W, seed, live):
    """x, w in {-1, 0, 1} on `live` input channels only, bias small integers: every running
    sum is an integer of magnitude <= 9 * len(live) <= 256, exact in bf16."""
    rng = np.random.default_rng(seed)
    x = np.zeros((B, Cin, H, W), np.float32)
    w = np.zeros((Cout, Cin, 3, 3), np.float32)
    x[:, live] = rng.integers(-1, 2, (B, len(live), H, W))
    w[:, live] = rng.integers(-1, 2, (Cout, len(live), 3, 3))
    b = rng.integers(-4, 5, Cout).astype(np.float32)
    return oracle.bf16_bits(x), oracle.bf16_bits(w), oracle.bf16_bits(b)


@pytest.mark.parametrize("B,Cin,Cout,H,W,live", [
    (2, 16, 8, 5, 7, list(range(16))),
    (1, 72, 10, 6, 4, [0, 5, 9, 17, 33, 62, 63, 64, 65, 66, 68, 70, 71, 3, 40, 50]),  # two chunks
    (1, 130, 3, 3, 3, [1, 2, 64, 65, 128, 129]),                                      # three chunks
])
def test_conv_with_exact_sums_is_the_exact_conv(B, Cin, Cout, H, W, live):
    xb, wb, bb = _small_int_case(B, Cin, Cout, H, W, Cin + H, live)
    y = oracle.bf16_value(oracle.conv3x3_bfp16_emul(xb, wb, bb)).astype(np.float64)
    np.testing.assert_array_equal(y, oracle.conv3x3_fwd(xb, wb, bb))
    rng = np.random.default_rng(1)
    dy = oracle.bf16_bits(rng.integers(-1, 2, (B, Cout, H, W)).astype(np.float32))
    gx = oracle.bf16_value(oracle.conv3x3_dgrad_bfp16_emul(dy, wb)).astype(np.float64)
    np.testing.assert_array_equal(gx, oracle.conv3x3_dgrad(dy, wb))


def _gate_quant(x, dim):
    """The gate's float formulation of the quantization (bfp16_training_gate.py:33-44)."""
    xf = x.float().movedim(dim, -1)
    shape = xf.shape
    blk = xf.reshape(*shape[:-1], shape[-1] // 8, 8)
    maxabs = blk.abs().amax(-1, keepdim=True)
    exp = torch.floor(torch.log2(maxabs.clamp_min(1e-38)))
    lsb = torch.exp2(exp - 6)
    q = torch.clamp(torch.round(blk / lsb), -128, 127) * lsb
    q = torch.where(maxabs > 0, q, torch.zeros_like(q))
    return q.reshape(shape).movedim(-1, dim)


def _gate_conv(x, w, chunk=64):
    """The gate's emulated conv (bfp16_training_gate.py:51-62): K order (tap, c), the
    running sum rounded to bf16 after every 64 columns."""
    B, C, H, W = x.shape
    xq = _gate_quant(x, 1)
    wq = _gate_quant(w.permute(0, 2, 3, 1).reshape(w.shape[0], -1), 1)
    cols = F.unfold(xq, 3, padding=1).reshape(B, C, 9, H * W).permute(0, 3, 2, 1).reshape(B * H * W, 9 * C)
    acc = torch.zeros(B * H * W, w.shape[0])
    for k0 in range(0, 9 * C, chunk):
        acc = (acc + cols[:, k0:k0 + chunk] @ wq[:, k0:k0 + chunk].t()).bfloat16().float()
    return acc.reshape(B, H, W, -1).permute(0, 3, 1, 2).contiguous()


@pytest.mark.parametrize("B,Cout,H,W", [(2, 40, 9, 9), (1, 64, 12, 7)])
def test_matches_the_reference_gate_formulation_at_64_channels(B, Cout, H, W):
    g = torch.Generator().manual_seed(B * 100 + Cout)
    x = torch.randn(B, 64, H, W, generator=g).bfloat16()
    w = (torch.randn(Cout, 64, 3, 3, generator=g) * 0.05).bfloat16()
    b = (torch.randn(Cout, generator=g) * 0.1).bfloat16()
    want = (_gate_conv(x.float(), w.float()) + b.float().view(1, -1, 1, 1)).bfloat16()
    got = oracle.conv3x3_bfp16_emul(_bits(x), _bits(w), _bits(b))
    np.testing.assert_array_equal(got, _bits(want))
    # input gradient (64 input channels of the gradient conv = 64 output channels here)
    w2 = (torch.randn(64, Cout, 3, 3, generator=g) * 0.05).bfloat16()
    dy = torch.randn(B, 64, H, W, generator=g).bfloat16()
    want_dx = _gate_conv(dy.float(), w2.flip(2, 3).transpose(0, 1).float()).bfloat16()
    np.testing.assert_array_equal(oracle.conv3x3_dgrad_bfp16_emul(_bits(dy), _bits(w2)), _bits(want_dx))


def test_error_size_against_the_exact_conv():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 128, 10, 10, generator=g).bfloat16()
    w = (torch.randn(96, 128, 3, 3, generator=g) * 0.03).bfloat16()
    exact = oracle.conv3x3_fwd(_bits(x), _bits(w))
    emul = oracle.bf16_value(oracle.conv3x3_bfp16_emul(_bits(x), _bits(w))).astype(np.float64)
    one = oracle.bf16_value(oracle.bf16_bits(exact.astype(np.float32))).astype(np.float64)
    rel = np.linalg.norm(emul - exact) / np.linalg.norm(exact)
    rel_one = np.linalg.norm(one - exact) / np.linalg.norm(exact)
    assert 2 * rel_one < rel < 0.05, (rel, rel_one)
