"""Writes tests/golden/bfp16_golden.json: SHA-256 digests of the reference's own BFP16
weight encoding (forward and dX forms) on seeded weights.

The producer is the reference's ``xdna_train/_native/conv_pack.cpp`` compiled in place
into ``oracle/_ref/conv_pack.so`` (``make -C oracle ref``; needs /root/reference, i.e.
this container only).  Channel counts are those of the reference's layout test
(tests/run_conv3x3w_pack.py:108-110) and the weight values follow its recipe
(:63-67): N(0,1) scaled per (co, ci) by 1e-3, 1 or 50, 30 % zeros at tap (0, 0), exact
ties at 1/8 steps at tap (1, 1), the first min(Cin, 8) input channels all zero.  Two
more cases carry special values (+-inf, NaN, bf16 subnormals, +-0) and every bf16 bit
pattern.  Weights are regenerated from the seed on both sides (``bfp16_weights``).
Run: ``python tests/golden/make_bfp16_golden.py``.
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(REPO))
import oracle  # noqa: E402

# (Cin, Cout, kind)
CASES = [(256, 128, "recipe"), (64, 64, "recipe"), (195, 64, "recipe"), (128, 128, "recipe"),
         (256, 256, "recipe"), (3, 10, "recipe"), (70, 130, "special"), (64, 1024, "allbits")]


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def bfp16_weights(cin: int, cout: int, kind: str, seed: int) -> np.ndarray:
    """OIHW bf16 bit patterns of one case."""
    rng = np.random.default_rng(seed)
    if kind == "allbits":
        # every bf16 pattern once (cout * cin * 9 >= 65536), in a seeded order
        n = cout * cin * 9
        bits = np.resize(rng.permutation(65536).astype(np.uint16), n)
        return bits.reshape(cout, cin, 3, 3)
    w = (rng.standard_normal((cout, cin, 3, 3)) * rng.choice([1e-3, 1, 50], (cout, cin, 1, 1))).astype(np.float32)
    w[:, :, 0, 0] = np.where(rng.random((cout, cin)) < 0.3, 0, w[:, :, 0, 0])
    w[:, :, 1, 1] = rng.integers(-40, 40, (cout, cin)) / 8.0
    w[:, : min(cin, 8), :, :] = 0
    bits = oracle.bf16_bits(w)
    if kind == "special":
        flat = bits.reshape(-1)
        pos = rng.choice(flat.size, 64, replace=False)
        specials = np.array([0x7F80, 0xFF80, 0x7FC0, 0xFFC1, 0x0001, 0x807F, 0x0000, 0x8000], np.uint16)
        flat[pos] = np.resize(specials, 64)
    return bits


def main() -> None:
    ref = oracle.ref_pack()
    if ref is None:
        sys.exit("oracle/_ref/conv_pack.so is missing: run `make -C oracle ref` where /root/reference exists")
    out = []
    for i, (cin, cout, kind) in enumerate(CASES):
        seed = 2000 + i
        w = np.ascontiguousarray(bfp16_weights(cin, cout, kind, seed))
        chunks = -(-cin // 64)
        fwd = []
        for nb in range(-(-cout // 128)):
            buf = np.zeros(chunks * oracle.BFP16_BYTES_PER_CHUNK, np.uint8)
            ref.xdna_conv3x3w_pack_weights_bfp16(w.ctypes.data, buf.ctypes.data, cout, cin, chunks, nb)
            fwd.append(sha(buf))
        dx_chunks = -(-cout // 64)
        dx = []
        for nb in range(-(-cin // 128)):
            buf = np.zeros(dx_chunks * oracle.BFP16_BYTES_PER_CHUNK, np.uint8)
            ref.xdna_conv3x3w_pack_weights_dx_bfp16(w.ctypes.data, buf.ctypes.data, cout, cin, dx_chunks, nb)
            dx.append(sha(buf))
        out.append({"cin": cin, "cout": cout, "kind": kind, "seed": seed, "fwd": fwd, "dx": dx})
    path = Path(__file__).parent / "bfp16_golden.json"
    path.write_text(json.dumps({"producer": "reference conv_pack.cpp (oracle/_ref)", "cases": out}, indent=1) + "\n")
    print(f"wrote {path} ({len(out)} cases)")


if __name__ == "__main__":
    main()
