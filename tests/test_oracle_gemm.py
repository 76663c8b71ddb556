"""The GEMM oracle (oracle.gemm: alpha * A.B + beta * bias in float64 of bf16 values) is
pinned by a pure-Python triple loop on small products, closed forms (identity and
permutation matrices, rank-one products, a zero operand), the bias/alpha/beta terms and
batched broadcasting.  A transposed operand or a dropped bias term fails one of these."""
import numpy as np
import pytest

import oracle


def _brute(a, b, bias=None, alpha=1.0, beta=1.0):
    av, bv = oracle.bf16_value(a).astype(float), oracle.bf16_value(b).astype(float)
    M, K = av.shape
    N = bv.shape[1]
    out = np.zeros((M, N))
    for i in range(M):
        for j in range(N):
            s = 0.0
            for k in range(K):
                s += float(av[i, k]) * float(bv[k, j])
            out[i, j] = alpha * s
    if bias is not None:
        out += beta * oracle.bf16_value(bias).astype(float)
    return out


@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (3, 5, 7), (8, 3, 2), (5, 16, 9)])
def test_matches_brute_force(M, K, N):
    rng = np.random.default_rng(M * 100 + K * 10 + N)
    a = oracle.rng_bf16(rng, (M, K))
    b = oracle.rng_bf16(rng, (K, N))
    bias = oracle.rng_bf16(rng, (N,))
    np.testing.assert_allclose(oracle.gemm(a, b), _brute(a, b), rtol=1e-13, atol=1e-13)
    np.testing.assert_allclose(oracle.gemm(a, b, bias, alpha=2.0, beta=0.5), _brute(a, b, bias, 2.0, 0.5),
                               rtol=1e-13, atol=1e-13)
    # beta = 0 drops the bias term
    np.testing.assert_allclose(oracle.gemm(a, b, bias, beta=0.0), _brute(a, b), rtol=1e-13, atol=1e-13)


def test_closed_forms():
    rng = np.random.default_rng(1)
    a = oracle.rng_bf16(rng, (6, 6))
    eye = oracle.bf16_bits(np.eye(6))
    av = oracle.bf16_value(a).astype(float)
    assert np.array_equal(oracle.gemm(a, eye), av)
    assert np.array_equal(oracle.gemm(eye, a), av)
    perm = np.eye(6)[[2, 0, 5, 1, 4, 3]]
    # P.A permutes rows, A.P permutes columns: a transposed operand would swap them
    assert np.array_equal(oracle.gemm(oracle.bf16_bits(perm), a), perm @ av)
    assert np.array_equal(oracle.gemm(a, oracle.bf16_bits(perm)), av[:, [1, 3, 0, 5, 4, 2]])
    # rank one: u v^T
    u = oracle.rng_bf16(rng, (4, 1))
    v = oracle.rng_bf16(rng, (1, 5))
    np.testing.assert_array_equal(oracle.gemm(u, v), np.outer(oracle.bf16_value(u), oracle.bf16_value(v)))
    assert not oracle.gemm(np.zeros((3, 4), np.uint16), oracle.rng_bf16(rng, (4, 2))).any()


def test_batched_matches_per_matrix():
    rng = np.random.default_rng(2)
    a = oracle.rng_bf16(rng, (3, 4, 5))
    b = oracle.rng_bf16(rng, (3, 5, 2))
    out = oracle.gemm(a, b)
    for i in range(3):
        np.testing.assert_allclose(out[i], _brute(a[i], b[i]), rtol=1e-13, atol=1e-13)
