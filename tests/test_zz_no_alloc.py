"""xdna_gemm_bf16_noalloc (for callers that cannot allocate: graph capture, serving
loops) against xdna_gemm_bf16 through the C ABI: the same bits on products whose split-K
partials use the library's device scratch, on two calls in a row with the second one
smaller (the scratch keeps the first call's partials), for both split-K kernels.  Also:
a product whose partials exceed the scratch is refused before anything runs, and the
entry point makes no allocation of the library's caching allocator."""
import ctypes

import pytest
import torch

from xdna_train import hip_abi

pytestmark = pytest.mark.gpu

SCRATCH = 64 << 20


def _stats(hip):
    arr = (ctypes.c_int64 * 6)()
    hip.xdna_hip_cache_stats(arr, 6)
    return list(arr)


def _operands(batch, M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    a = (torch.randn(batch, M, K, generator=g) * 0.5).bfloat16().cuda()
    b = (torch.randn(batch, K, N, generator=g) * 0.5).bfloat16().cuda()
    bias = torch.randn(N, generator=g).bfloat16().cuda()
    return a, b, bias


def _gemm(fn, a, b, bias, stream, alpha=1.0, beta=0.0):
    batch, M, K = a.shape
    N = b.shape[2]
    c = torch.full((batch, M, N), -7.0, device="cuda").bfloat16()  # no stale zeros help
    rc = fn(a.data_ptr(), b.data_ptr(), c.data_ptr(), bias.data_ptr() if beta else None, batch, M, N, K,
            K, 1, M * K, N, 1, K * N, N, 1, M * N, 1 if beta else 0, 0, 1, alpha, beta, stream)
    assert rc == 0, hip_abi.last_error()
    return c


def _split_bytes(batch, M, N, K):
    """The split-K partial bytes the large-tile path plans for a product it takes (host
    copy of the launcher's rule, used only to pick a refused shape)."""
    tiles2 = -(-N // 256) * -(-M // 256) * batch
    kt2 = -(-K // 64)
    if not (tiles2 < 256 and kt2 >= 8):
        return 0
    sp = max(1, min(kt2 // 4, -(-256 // tiles2), 65535 // batch))
    kt_per = -(-kt2 // sp)
    nsplit = -(-kt2 // kt_per)
    return nsplit * batch * M * N * 4 if nsplit > 1 else 0


# (batch, M, N, K): the first of each pair fills much of the scratch, the second is smaller
PAIRS = [
    ((1, 512, 384, 16384), (1, 256, 128, 16384)),  # 256 x 256 four-wave kernel, split-K
    ((1, 768, 768, 8192), (1, 256, 256, 2048)),    # 128 x 128 kernel, split-K over blockIdx.z
    ((4, 64, 64, 8192), (2, 64, 96, 4096)),        # batched
]


@pytest.mark.parametrize("first,second", PAIRS, ids=["large_tiles", "small_tiles", "batched"])
def test_noalloc_matches_gemm_on_two_calls(hip, stream, first, second):
    print("noalloc gemm", first, second, flush=True)
    for i, (shape, beta) in enumerate(((first, 0.0), (second, 1.0))):
        a, b, bias = _operands(*shape, seed=10 + i)
        torch.cuda.synchronize()
        s0 = _stats(hip)
        ref = _gemm(hip.xdna_gemm_bf16, a, b, bias, stream, alpha=1.0, beta=beta)
        torch.cuda.synchronize()
        s1 = _stats(hip)
        # the allocating entry point takes a cache block for the partials: split-K ran
        assert sum(s1[3:5]) > sum(s0[3:5]), f"{shape} did not take the split-K path"
        got = _gemm(hip.xdna_gemm_bf16_noalloc, a, b, bias, stream, alpha=1.0, beta=beta)
        torch.cuda.synchronize()
        s2 = _stats(hip)
        # no allocation of the caching allocator (fresh blocks and reuses unchanged)
        assert s2[3:5] == s1[3:5], (s1, s2)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"call {i} {shape}"


def test_noalloc_refuses_partials_beyond_the_scratch(hip, stream):
    shape = (1, 3840, 3840, 512)
    assert _split_bytes(*shape) > SCRATCH
    a, b, bias = _operands(*shape, seed=3)
    c = torch.zeros(1, 3840, 3840, device="cuda").bfloat16()
    torch.cuda.synchronize()
    n0 = hip.xdna_hip_launch_count()
    rc = hip.xdna_gemm_bf16_noalloc(a.data_ptr(), b.data_ptr(), c.data_ptr(), None, 1, 3840, 3840, 512,
                                    512, 1, 0, 3840, 1, 0, 3840, 1, 0, 0, 0, 0, 1.0, 0.0, stream)
    assert rc == -1
    msg = hip_abi.last_error()
    assert "scratch" in msg and "xdna_gemm_bf16_noalloc" in msg
    torch.cuda.synchronize()
    assert not c.view(torch.int16).any()  # nothing ran
    assert hip.xdna_hip_launch_count() - n0 <= 1  # the admitted launch count, no kernels
    # the same product through the allocating entry point works
    assert hip.xdna_gemm_bf16(a.data_ptr(), b.data_ptr(), c.data_ptr(), None, 1, 3840, 3840, 512,
                              512, 1, 0, 3840, 1, 0, 3840, 1, 0, 0, 0, 0, 1.0, 0.0, stream) == 0
    torch.cuda.synchronize()
    ref = (a[0].float() @ b[0].float())
    got = c[0].float()
    assert float((got - ref).abs().max()) <= float(ref.abs().max()) * 2 ** -6
    # a product without split-K needs no scratch at all
    a2, b2, bias2 = _operands(1, 512, 512, 256, seed=4)
    ref2 = _gemm(hip.xdna_gemm_bf16, a2, b2, bias2, stream)
    got2 = _gemm(hip.xdna_gemm_bf16_noalloc, a2, b2, bias2, stream)
    torch.cuda.synchronize()
    assert torch.equal(got2.view(torch.int16), ref2.view(torch.int16))
