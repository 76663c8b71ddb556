"""HIP bf16 GEMM vs float64 products of the bf16 operands (oracle.gemm).

Covers the operand layouts Linear produces (forward: B = W^T, k-contiguous; dX:
B = W, n-contiguous; dW: A = dY^T, m-contiguous), element-stride views that force the
scalar staging path, ragged sizes, K = 0, the addmm bias forms and alpha/beta, and
batched products (bmm).  Bar: 2 bf16 ulp (floored) and rel L2 <= 1e-2.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import check_bf16, dev, dev_zeros, host, ptr, stream

pytestmark = pytest.mark.gpu


def _mat(rng, r, c, scale=1.0):
    return oracle.rng_bf16(rng, (r, c), scale)


def _run(hip, a_t, b_t, M, N, K, a_s, b_s, bias=None, bias_mode=0, bias_s=(0, 0), alpha=1.0,
         beta=0.0, batch=1, sa=0, sb=0):
    c = dev_zeros((batch, M, N))
    rc = hip.xdna_gemm_bf16(ptr(a_t), ptr(b_t), ptr(c), ptr(bias), batch, M, N, K, a_s[0], a_s[1], sa,
                            b_s[0], b_s[1], sb, N, 1, M * N, bias_mode, bias_s[0], bias_s[1], alpha,
                            beta, stream())
    assert rc == 0
    return host(c)


@pytest.fixture
def variant(hip, request):
    assert hip.xdna_gemm_set_variant(request.param) == 0
    yield request.param
    assert hip.xdna_gemm_set_variant(0) == 0


# kernel variants (xdna_gemm_set_variant): 128 x 128 tiles, 256 x 256 tiles (eight- and four-wave,
# four-wave with direct-to-LDS loads, and that with 16x16x32 MFMAs)
@pytest.mark.parametrize("variant", [1, 2, 3, 4, 5], indirect=True, ids=lambda v: f"v{v}")
@pytest.mark.parametrize("M,N,K", [(256, 384, 512), (130, 70, 33), (1, 1, 1), (64, 257, 8),
                                   (300, 128, 1000), (520, 264, 136)])
@pytest.mark.parametrize("layout", ["nn", "nt", "tn", "tt"])
def test_layouts(hip, M, N, K, layout, variant):
    print(f"gemm {layout} {M}x{N}x{K} variant {variant}", flush=True)
    rng = np.random.default_rng(M + N + K)
    a = _mat(rng, M, K)
    b = _mat(rng, K, N)
    ref = oracle.gemm(a, b)
    # store A as [M][K] (n) or as A^T [K][M] (t); same for B
    if layout[0] == "n":
        da, a_s = dev(a), (K, 1)
    else:
        da, a_s = dev(np.ascontiguousarray(a.T)), (1, M)
    if layout[1] == "n":
        db, b_s = dev(b), (N, 1)
    else:
        db, b_s = dev(np.ascontiguousarray(b.T)), (1, K)
    got = _run(hip, da, db, M, N, K, a_s, b_s)[0]
    check_bf16(got, ref, what=f"gemm {layout} {M}x{N}x{K}")


def test_strided_views_scalar_path(hip):
    rng = np.random.default_rng(1)
    M, N, K = 70, 50, 40
    big_a = _mat(rng, M, 2 * K + 1)
    big_b = _mat(rng, K, 3 * N)
    a = big_a[:, 1:2 * K + 1:2]
    b = big_b[:, ::3]
    ref = oracle.gemm(a, b)
    da, db = dev(big_a), dev(big_b)
    c = dev_zeros((M, N))
    rc = hip.xdna_gemm_bf16(ptr(da) + 2, ptr(db), ptr(c), None, 1, M, N, K, 2 * K + 1, 2, 0, 3 * N, 3, 0,
                            N, 1, 0, 0, 0, 0, 1.0, 0.0, stream())
    assert rc == 0
    check_bf16(host(c), ref, what="strided")


def test_k_zero_gives_beta_bias(hip):
    rng = np.random.default_rng(2)
    M, N = 5, 7
    bias = oracle.rng_bf16(rng, (N,))
    c = dev_zeros((M, N))
    rc = hip.xdna_gemm_bf16(ptr(dev_zeros((1,))), ptr(dev_zeros((1,))), ptr(c), ptr(dev(bias)), 1, M, N, 0,
                            0, 1, 0, 1, 0, 0, N, 1, 0, 1, 0, 1, 1.0, 2.0, stream())
    assert rc == 0
    np.testing.assert_array_equal(oracle.bf16_value(host(c)), np.broadcast_to(2 * oracle.bf16_value(bias), (M, N)))


@pytest.mark.parametrize("variant", [1, 2, 3, 4, 5], indirect=True, ids=lambda v: f"v{v}")
@pytest.mark.parametrize("mode", [1, 2, 3])
def test_bias_modes_alpha_beta(hip, mode, variant):
    rng = np.random.default_rng(3 + mode)
    M, N, K = 96, 160, 64
    a, b = _mat(rng, M, K), _mat(rng, K, N)
    if mode == 1:
        bias, bs, shape = oracle.rng_bf16(rng, (N,)), (0, 1), (N,)
    elif mode == 2:
        bias, bs, shape = oracle.rng_bf16(rng, (M, N)), (N, 1), (M, N)
    else:
        bias, bs, shape = oracle.rng_bf16(rng, (M,)), (1, 0), (M, 1)
    alpha, beta = 0.5, -1.5
    ref = oracle.gemm(a, b, bias.reshape(shape), alpha=alpha, beta=beta)
    got = _run(hip, dev(a), dev(b), M, N, K, (K, 1), (N, 1), bias=dev(bias), bias_mode=mode, bias_s=bs,
               alpha=alpha, beta=beta)[0]
    check_bf16(got, ref, what=f"bias mode {mode}")


@pytest.mark.parametrize("variant", [1, 2, 3, 4, 5], indirect=True, ids=lambda v: f"v{v}")
def test_batched(hip, variant):
    rng = np.random.default_rng(5)
    Bt, M, N, K = 6, 40, 72, 96
    a = oracle.rng_bf16(rng, (Bt, M, K))
    b = oracle.rng_bf16(rng, (Bt, K, N))
    ref = oracle.gemm(a, b)
    got = _run(hip, dev(a), dev(b), M, N, K, (K, 1), (N, 1), batch=Bt, sa=M * K, sb=K * N)
    check_bf16(got, ref, what="bmm")
    # Gram form used by style losses: F . F^T with F [B][C][HW]
    f = oracle.rng_bf16(rng, (Bt, 32, 81))
    ref_g = oracle.gemm(f, np.swapaxes(f, 1, 2))
    got_g = _run(hip, dev(f), dev(f), 32, 32, 81, (81, 1), (1, 81), batch=Bt, sa=32 * 81, sb=32 * 81)
    check_bf16(got_g, ref_g, what="gram")


@pytest.mark.parametrize("variant", [1, 2, 3, 4, 5], indirect=True, ids=lambda v: f"v{v}")
def test_mlp_shape(hip, variant):
    """One of config 3's GEMMs (x [8192,1024] . W^T [1024,4096]) on a row subset."""
    rng = np.random.default_rng(6)
    M, N, K = 512, 4096, 1024
    a = _mat(rng, M, K)
    w = _mat(rng, N, K, 0.03)
    ref = oracle.gemm(a, w.T)
    got = _run(hip, dev(a), dev(w), M, N, K, (K, 1), (1, K))[0]
    check_bf16(got, ref, what="mlp fwd")


@pytest.mark.parametrize("bias_mode", [0, 2])
def test_gram_split_k(hip, bias_mode):
    """Batched Gram products (few output tiles, long K): the split-K path, whose fp32
    partials are summed in split order, with alpha, beta and a matrix bias term."""
    print(f"gemm gram split-k bias_mode {bias_mode}", flush=True)
    rng = np.random.default_rng(11)
    batch, C, HW = 3, 64, 1296
    f = oracle.rng_bf16(rng, (batch, C, HW))
    bias = oracle.rng_bf16(rng, (C, C)) if bias_mode else None
    alpha, beta = 0.5, 1.0
    da = dev(f)
    got = _run(hip, da, da, C, C, HW, (HW, 1), (1, HW), bias=dev(bias) if bias_mode else None,
               bias_mode=bias_mode, bias_s=(C, 1) if bias_mode else (0, 0), alpha=alpha, beta=beta,
               batch=batch, sa=C * HW, sb=C * HW)
    for i in range(batch):
        ref = alpha * oracle.gemm(f[i], np.ascontiguousarray(f[i].T))
        if bias_mode:
            ref = ref + beta * oracle.bf16_value(bias).astype(np.float64)
        check_bf16(got[i], ref, what=f"gram split-k batch {i}")
    # fixed-order split reduction: identical on a second run
    again = _run(hip, da, da, C, C, HW, (HW, 1), (1, HW), bias=dev(bias) if bias_mode else None,
                 bias_mode=bias_mode, bias_s=(C, 1) if bias_mode else (0, 0), alpha=alpha, beta=beta,
                 batch=batch, sa=C * HW, sb=C * HW)
    assert np.array_equal(got, again)


@pytest.mark.parametrize("M,N,K,bias_mode", [(2048, 1024, 4096, 0), (2048, 1024, 4096, 1), (512, 260, 8192, 3),
                                             (8192, 1024, 4096, 1)])
def test_split_k_epilogue_forms_agree(hip, M, N, K, bias_mode):
    """Products with split-K partials (few output tiles, long K): the four-wide epilogue
    (row-major C, N % 4 == 0) and the element form (C written transposed, column stride M)
    give the same bits, and both meet the bar against the oracle where it is cheap."""
    rng = np.random.default_rng(M + N + K + bias_mode)
    a = _mat(rng, M, K)
    b = _mat(rng, K, N)
    da, db = dev(a), dev(b)
    blen = N if bias_mode == 1 else M
    bias = oracle.rng_bf16(rng, (blen,), 0.5)
    dbias = dev(bias)
    bs = (0, 1) if bias_mode == 1 else (1, 0)
    c1 = dev_zeros((M, N))
    c2 = dev_zeros((N, M))
    for c, cm, cn in ((c1, N, 1), (c2, 1, M)):
        assert hip.xdna_gemm_bf16(ptr(da), ptr(db), ptr(c), ptr(dbias) if bias_mode else None, 1, M, N, K, K, 1,
                                  0, N, 1, 0, cm, cn, 0, bias_mode, bs[0], bs[1], 1.0, 1.0, stream()) == 0
    g1, g2 = host(c1), host(c2).T
    np.testing.assert_array_equal(g1, g2)
    if M * N * K <= 2048 * 1024 * 4096:
        ref = oracle.gemm(a[:256], b)
        if bias_mode == 1:
            ref = ref + oracle.bf16_value(bias)[None, :]
        elif bias_mode == 3:
            ref = ref + oracle.bf16_value(bias)[:256, None]
        check_bf16(g1[:256], ref, what=f"split-K {M}x{N}x{K}")


@pytest.mark.parametrize("M,N,K,bias_mode", [(4096, 4096, 1024, 1), (4100, 4100, 1024, 3), (4104, 4096, 1056, 2),
                                             (4096, 4104, 1024, 0)])
def test_large_tile_epilogue_bias_forms(hip, M, N, K, bias_mode):
    """The 256 x 256 kernel without split-K, whose epilogue is compiled per bias form (none,
    per column, any other): row-major C and the same product written transposed (column
    stride M) give the same bits for every bias form, with alpha, beta and ragged M and N;
    the first rows meet the bar against the oracle."""
    print(f"gemm epilogue forms {M}x{N}x{K} bias {bias_mode}", flush=True)
    rng = np.random.default_rng(M + 3 * N + K + bias_mode)
    a = _mat(rng, M, K)
    b = _mat(rng, K, N, 0.05)
    da, db = dev(a), dev(b)
    if bias_mode == 1:
        bias, bs = oracle.rng_bf16(rng, (N,)), (0, 1)
    elif bias_mode == 2:
        bias, bs = oracle.rng_bf16(rng, (M, N)), (N, 1)
    else:
        bias, bs = oracle.rng_bf16(rng, (M,)), (1, 0)
    dbias = dev(bias)
    c1 = dev_zeros((M, N))
    c2 = dev_zeros((N, M))
    for c, cm, cn in ((c1, N, 1), (c2, 1, M)):
        assert hip.xdna_gemm_bf16(ptr(da), ptr(db), ptr(c), ptr(dbias) if bias_mode else None, 1, M, N, K, K, 1,
                                  0, N, 1, 0, cm, cn, 0, bias_mode, bs[0], bs[1], 0.5, -1.0, stream()) == 0
    g1, g2 = host(c1), host(c2).T
    np.testing.assert_array_equal(g1, g2)
    ref = 0.5 * oracle.gemm(a[:64], b)
    if bias_mode == 1:
        ref = ref - oracle.bf16_value(bias)[None, :]
    elif bias_mode == 2:
        ref = ref - oracle.bf16_value(bias)[:64]
    elif bias_mode == 3:
        ref = ref - oracle.bf16_value(bias)[:64, None]
    check_bf16(g1[:64], ref, what=f"epilogue forms {M}x{N}x{K}")
