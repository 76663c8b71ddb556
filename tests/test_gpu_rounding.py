"""The bf16 rounding every kernel applies (f32_to_bf16: gfx950's v_cvt_pk_bf16_f32 plus a
NaN select) against round-to-nearest-even computed with integer arithmetic, over all
2^32 fp32 bit patterns: identical for every non-NaN input (subnormals included); every
NaN gives 0x7FC0 (c10::BFloat16's convention)."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_bf16_rounding_all_patterns(hip):
    chunk = 1 << 28
    out = torch.empty(chunk, dtype=torch.int16, device="cuda")
    for c in range(1 << 32 >> 28):
        print(f"bf16 rounding chunk {c}", flush=True)
        u = torch.arange(c * chunk, (c + 1) * chunk, dtype=torch.int64, device="cuda")
        bits = (u - (1 << 32) * (u >= (1 << 31))).to(torch.int32)  # two's complement view
        f = bits.view(torch.float32)
        assert hip.xdna_round_bf16(f.data_ptr(), out.data_ptr(), chunk,
                                   torch.cuda.current_stream().cuda_stream) == 0
        # reference: (u + 0x7FFF + ((u >> 16) & 1)) >> 16 on the unsigned pattern
        lsb = (u >> 16) & 1
        ref = ((u + 0x7FFF + lsb) >> 16) & 0xFFFF
        nan = (u & 0x7FFFFFFF) > 0x7F800000
        ref = torch.where(nan, torch.full_like(ref, 0x7FC0), ref)
        got = out.to(torch.int64) & 0xFFFF
        bad = int((got != ref).sum())
        assert bad == 0, f"chunk {c}: {bad} mismatches"
        del u, bits, f, lsb, ref, nan, got
