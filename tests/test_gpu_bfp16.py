"""HIP BFP16 weight codec vs the oracle and the reference digests: bit-exact.

Cases: every golden case (the reference layout test's channel counts and weight recipe,
special values, every bf16 bit pattern), forward and dX forms, each 128-channel block;
a buffer reused across shapes (every byte is written); the decode kernel against the
oracle's decode; argument errors.
"""
import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from gpu_util import dev, host, ptr, stream

sys.path.insert(0, str(Path(__file__).parent / "golden"))
from make_bfp16_golden import bfp16_weights  # noqa: E402

pytestmark = pytest.mark.gpu

GOLDEN = json.loads((Path(__file__).parent / "golden" / "bfp16_golden.json").read_text())["cases"]


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _bytes(t):
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.uint8)


@pytest.mark.parametrize("case", GOLDEN, ids=lambda c: f"ci{c['cin']}co{c['cout']}{c['kind']}")
def test_weights_golden(hip, case):
    cin, cout = case["cin"], case["cout"]
    print(f"bfp16 weights cin {cin} cout {cout} {case['kind']}", flush=True)
    w = bfp16_weights(cin, cout, case["kind"], case["seed"])
    dw = dev(w)
    chunks = -(-cin // 64)
    n = hip.xdna_conv3x3w_weights_bfp16_bytes(chunks)
    assert n == chunks * oracle.BFP16_BYTES_PER_CHUNK
    # one buffer for every block, filled with 0xAB first: the kernel writes every byte
    out = torch.full((n,), 0xAB, dtype=torch.uint8, device="cuda")
    for nb, digest in enumerate(case["fwd"]):
        assert hip.xdna_conv3x3w_pack_weights_bfp16(ptr(dw), ptr(out), cout, cin, chunks, nb, stream()) == 0
        got = _bytes(out)
        assert _sha(got) == digest, f"fwd block {nb}"
        np.testing.assert_array_equal(got, oracle.pack_weights_bfp16(w, chunks, nb))
    dchunks = -(-cout // 64)
    nd = hip.xdna_conv3x3w_weights_bfp16_bytes(dchunks)
    outd = torch.full((nd,), 0xCD, dtype=torch.uint8, device="cuda")
    for nb, digest in enumerate(case["dx"]):
        assert hip.xdna_conv3x3w_pack_weights_dx_bfp16(ptr(dw), ptr(outd), cout, cin, dchunks, nb, stream()) == 0
        assert _sha(_bytes(outd)) == digest, f"dx block {nb}"


def test_decode_matches_oracle(hip):
    rng = np.random.default_rng(3)
    blocks = rng.integers(0, 256, (4099, 9), dtype=np.uint8)
    blocks[:, 0] = rng.integers(100, 160, 4099)          # normal fp32 results
    src = torch.from_numpy(blocks.reshape(-1).copy()).cuda()
    dst = torch.empty(4099 * 8, dtype=torch.float32, device="cuda")
    assert hip.xdna_bfp16_decode_f32(ptr(src), ptr(dst), 4099, stream()) == 0
    np.testing.assert_array_equal(host(dst).astype(np.float64), oracle.bfp16_decode(blocks))


def test_round_trip_within_half_step(hip):
    rng = np.random.default_rng(4)
    w = oracle.bf16_bits(rng.standard_normal((128, 64, 3, 3)).astype(np.float32))
    out = torch.empty(hip.xdna_conv3x3w_weights_bfp16_bytes(1), dtype=torch.uint8, device="cuda")
    assert hip.xdna_conv3x3w_pack_weights_bfp16(ptr(dev(w)), ptr(out), 128, 64, 1, 0, stream()) == 0
    blk = _bytes(out).reshape(-1, 9)
    dec = torch.empty(blk.shape[0] * 8, dtype=torch.float32, device="cuda")
    assert hip.xdna_bfp16_decode_f32(ptr(out), ptr(dec), blk.shape[0], stream()) == 0
    # block order [tap][n16][k8][two][nl][kl] back to OIHW
    v = host(dec).astype(np.float64).reshape(9, 8, 8, 2, 8, 8)
    back = v.transpose(1, 3, 4, 2, 5, 0).reshape(128, 64, 3, 3)
    step = np.ldexp(1.0, blk[:, 0].astype(np.int64) - 133).reshape(9, 8, 8, 2, 8, 1)
    step = np.broadcast_to(step, (9, 8, 8, 2, 8, 8)).transpose(1, 3, 4, 2, 5, 0).reshape(128, 64, 3, 3)
    m = blk[:, 1:].view(np.int8).reshape(9, 8, 8, 2, 8, 8).transpose(1, 3, 4, 2, 5, 0).reshape(128, 64, 3, 3)
    free = (m > -128) & (m < 127)
    err = np.abs(back - oracle.bf16_value(w))
    assert (err[free] <= step[free] / 2).all()


def test_argument_errors(hip):
    w = dev(np.zeros((4, 4, 3, 3), np.uint16))
    out = torch.empty(hip.xdna_conv3x3w_weights_bfp16_bytes(1) + 16, dtype=torch.uint8, device="cuda")
    assert hip.xdna_conv3x3w_pack_weights_bfp16(ptr(w), ptr(out), 0, 4, 1, 0, stream()) == -1
    assert hip.xdna_conv3x3w_pack_weights_bfp16(ptr(w), ptr(out) + 1, 4, 4, 1, 0, stream()) == -1
    assert "aligned" in hip.xdna_hip_last_error().decode()
    assert hip.xdna_conv3x3w_weights_bfp16_bytes(0) == 0
