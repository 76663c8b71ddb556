"""Wait states before MFMAs written as inline assembly (CPU test: compiles to gfx950 asm).

The 16x16x32 GEMM and conv rows kernels issue their MFMAs from inline-assembly statements,
which the compiler's hazard recognizer does not see.  A VALU instruction that writes a
register an MFMA then reads (operand A, B or the accumulator) needs 2 wait states before
that MFMA; those kernels rely on their operands coming straight from LDS reads and on an
explicit fence after the accumulators' initial values.  This test compiles the kernels'
sources to assembly with the build's flags and checks every MFMA of every kernel for a
VALU write of one of its operands within the 2 preceding wait states, and, after every
inline-assembly MFMA (between ``;;#ASMSTART`` and ``;;#ASMEND``), every other instruction
for a read or write of that MFMA's accumulator registers within the wait states an MFMA
result needs before anything but a chained MFMA may touch it (the compiler pads only the
MFMAs it generates itself; the kernels' fence pads the epilogue).
"""
import re
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(REPO / "pytorch-xdna2_amd"))
import build_native  # noqa: E402

SOURCES = ["gemm.hip", "conv3x3.hip"]
NEEDED = 2  # wait states between a VALU write and an MFMA reading the register
# wait states between an MFMA writing its accumulators and another instruction reading or
# writing them: the longest MFMA's figure (16 passes, 18 + 1), kept for every MFMA shape
AFTER = 19


def _regs(tok):
    m = re.match(r"([va])\[(\d+):(\d+)\]", tok)
    if m:
        return {(m.group(1), k) for k in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r"([va])(\d+)$", tok)
    return {(m.group(1), int(m.group(2)))} if m else set()


def hazards(asm_lines):
    """(line, writer, mfma) for every MFMA reading a register a VALU instruction wrote
    fewer than NEEDED wait states earlier (s_nop n counts n + 1)."""
    found, recent = [], []  # recent: (wait states, registers written, text)
    for n, line in enumerate(asm_lines):
        text = line.strip()
        if not text or text[0] in ";." or text.endswith(":"):
            continue  # labels keep the window: the textual predecessor falls through
        op, *rest = text.split()
        toks = [t.strip(",") for t in rest]
        if op.startswith("v_mfma"):
            reads = set().union(*(_regs(t) for t in toks[1:4]))
            ws = 0
            for w, dst, src in reversed(recent):
                if ws >= NEEDED:
                    break
                if dst & reads:
                    found.append((n, src, text))
                ws += w
        if op == "s_nop":
            recent.append((int(toks[0]) + 1, set(), text))
        else:
            writes_vgpr = op.startswith("v_") and not op.startswith(("v_mfma", "v_cmp", "v_readfirstlane",
                                                                       "v_readlane"))
            recent.append((1, _regs(toks[0]) if writes_vgpr and toks else set(), text))
        recent = recent[-8:]
    return found


def accumulator_hazards(asm_lines):
    """(line, mfma, reader) for every instruction other than an MFMA that reads or writes an
    accumulator register of an inline-assembly MFMA fewer than AFTER wait states after it
    (v_accvgpr copies in the k-loop, epilogue stores before the fence)."""
    found, recent, inline = [], [], False  # recent: (wait states, accumulator registers, text)
    for n, line in enumerate(asm_lines):
        text = line.strip()
        if ";;#ASMSTART" in text:
            inline = True
            continue
        if ";;#ASMEND" in text:
            inline = False
            continue
        if not text or text[0] in ";." or text.endswith(":"):
            continue
        op, *rest = text.split()
        toks = [t.strip(",") for t in rest]
        if op.startswith("v_mfma"):
            recent.append((1, _regs(toks[0]) if inline and toks else set(), text))
        elif op == "s_nop":
            recent.append((int(toks[0]) + 1, set(), text))
        else:
            touched = set().union(*(_regs(t) for t in toks)) if toks else set()
            ws = 0
            for w, acc, src in reversed(recent):
                if ws >= AFTER:
                    break
                if acc & touched:
                    found.append((n, src, text))
                    break
                ws += w
            recent.append((1, set(), text))
        recent = recent[-2 * AFTER:]
    return found


def test_scanner_finds_a_planted_hazard():
    asm = ["k:", "v_mov_b32_e32 v4, v1", "v_mfma_f32_16x16x32_bf16 a[0:3], v[4:7], v[8:11], a[0:3]",
           "s_nop 1", "v_mov_b32_e32 v9, v1", "s_nop 1", "v_mfma_f32_16x16x32_bf16 a[0:3], v[4:7], v[8:11], a[0:3]",
           "v_accvgpr_write_b32 a2, 0", "v_mfma_f32_16x16x32_bf16 a[0:3], v[4:7], v[8:11], a[0:3]"]
    got = hazards(asm)
    assert [g[0] for g in got] == [2, 8]


def test_accumulator_scanner_finds_planted_hazards():
    mfma = "v_mfma_f32_16x16x32_bf16 a[0:3], v[4:7], v[8:11], a[0:3]"
    asm = ["k:", ";;#ASMSTART", mfma, ";;#ASMEND", "v_accvgpr_read_b32 v1, a2",  # too soon: line 4
           ";;#ASMSTART", mfma, ";;#ASMEND", "s_nop 7", "s_nop 7", "s_nop 2",  # 19 wait states
           "global_store_dwordx4 v[0:1], a[0:3], off",
           ";;#ASMSTART", mfma, ";;#ASMEND", mfma,  # a chained MFMA is fine
           "v_accvgpr_write_b32 a1, 0",  # too soon after the inline one: line 16
           "s_nop 7", "s_nop 7", "s_nop 4",
           mfma, "v_accvgpr_read_b32 v1, a2"]  # a compiler-generated MFMA: not checked here
    got = accumulator_hazards(asm)
    assert [g[0] for g in got] == [4, 16]


@pytest.mark.skipif(not Path(build_native.HIPCC).exists() and shutil.which("hipcc") is None,
                    reason="hipcc not available")
@pytest.mark.parametrize("src", SOURCES)
def test_inline_mfma_operands_have_their_wait_states(src, tmp_path):
    out = tmp_path / (Path(src).stem + ".s")
    cmd = [build_native.HIPCC, *build_native.HIP_FLAGS, "--cuda-device-only", "-S",
           str(build_native.CSRC / src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stderr[-2000:]
    lines = out.read_text().split("\n")
    assert any("v_mfma_f32_16x16x32_bf16" in line for line in lines), "no 16x16x32 MFMA compiled"
    bad = hazards(lines)
    assert not bad, f"{len(bad)} MFMA operand hazards, first: {bad[:3]}"
    bad = accumulator_hazards(lines)
    assert not bad, f"{len(bad)} accumulator hazards after inline MFMAs, first: {bad[:3]}"
