"""Writes tests/golden/pack_golden.json: SHA-256 digests of the reference's own
conv3x3w host packing on seeded inputs.

The producer is the reference's ``xdna_train/_native/conv_pack.cpp`` compiled in place
into ``oracle/_ref/conv_pack.so`` (``make -C oracle ref``; needs /root/reference, i.e.
this container only).  The cases are the shapes of the reference's layout test
(tests/run_conv3x3w_pack.py:108-110 full layouts, :184-185 range cases, :244-246 strip
cases).  Inputs are regenerated from the seed on both sides:

    x   = bf16(rng.standard_normal((B, C, H, W)))        rng = np.random.default_rng(seed)
    raw = rng.integers(0, 65536, (groups*2048, 128))     drawn after x, same generator

Recorded per case: the packed input digest (buffer zero-filled, then packed once), with
halo_zero where strips exist, and the digest of the NCHW output of unpacking `raw`
into channels [c_start, c_start+min(Cout,128)) of a zeroed [B][Cout+c_extra][H][W].
Run: ``python tests/golden/make_pack_golden.py``.
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

FULL = [(40, 256, 36, 36, 128), (40, 64, 36, 36, 64), (4, 195, 36, 36, 64), (40, 128, 9, 9, 128),
        (40, 256, 18, 18, 256), (3, 3, 5, 7, 10)]
RANGE = [(3, 70, 5, 7, 10)]
STRIPS = [(2, 64, 8, 36, 64), (3, 64, 8, 37, 64), (2, 70, 9, 56, 10), (2, 64, 6, 64, 128),
          (2, 3, 7, 68, 64), (1, 64, 5, 69, 64), (3, 128, 4, 112, 128), (2, 64, 3, 224, 128),
          (2, 64, 5, 35, 64)]


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def inputs(seed, B, C, H, W, groups):
    rng = np.random.default_rng(seed)
    x = oracle.bf16_bits(rng.standard_normal((B, C, H, W)).astype(np.float32))
    raw = rng.integers(0, 65536, (groups * oracle.GROUP_OUT_ROWS, 128), dtype=np.uint16)
    return x, raw


def ref_case(ref, seed, B, C, H, W, Cout, strips, c_extra=3, c_start=2):
    S, So, Wg, wp, m_total, groups = oracle.geometry(B, H, W, strips)
    chunks = -(-C // 64)
    x, raw = inputs(seed, B, C, H, W, groups)
    rec = {"seed": seed, "B": B, "C": C, "H": H, "W": W, "Cout": Cout, "strips": strips,
           "S": S, "So": So, "wp": wp, "groups": groups, "chunks": chunks,
           "c_extra": c_extra, "c_start": c_start}
    for hz in ([0, 1] if S > 1 else [0]):
        dst = np.zeros((groups, chunks, oracle.GROUP_ROWS, 64), np.uint16)
        ref.xdna_conv3x3w_pack_input_strips_range_bf16(x.ctypes.data, dst.ctypes.data, B, C, H, W,
                                                       S, So, hz, chunks, 0, groups)
        rec[f"pack_h{hz}"] = sha(dst)
    nv = min(Cout, 128)
    out = np.zeros((B, Cout + c_extra, H, W), np.uint16)
    ref.xdna_conv3x3w_unpack_output_strips_range_bf16(raw.ctypes.data, out.ctypes.data, B, H, W, S,
                                                      So, nv, Cout + c_extra, c_start, 0, m_total)
    rec["unpack"] = sha(out)
    return rec


def main():
    ref = oracle.ref_pack()
    if ref is None:
        raise SystemExit("oracle/_ref/conv_pack.so missing: run `make -C oracle ref` where "
                         "/root/reference exists")
    ref.xdna_conv_set_threads(8)
    cases = []
    seed = 100
    for shp in FULL + RANGE:
        cases.append(ref_case(ref, seed, *shp, strips=False))
        seed += 1
    for shp in STRIPS:
        cases.append(ref_case(ref, seed, *shp, strips=True))
        seed += 1
    out = {"producer": "reference conv_pack.cpp built in oracle/_ref", "cases": cases}
    path = Path(__file__).with_name("pack_golden.json")
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {path} ({len(cases)} cases)")


if __name__ == "__main__":
    main()
