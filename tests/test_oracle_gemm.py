"""Pins oracle/gemm.py: exact int64 brute force for the per-group partials and
a float64 dequant_awq matmul (paroquant_marlin_w4a8.py:227-235) for the epilogue.
"""

import numpy as np
import pytest

from oracle import gemm


def _rand_case(rng, M, N, K):
    G = K // 128
    xq = rng.integers(-127, 128, (M, K)).astype(np.int8)
    codes = rng.integers(0, 16, (N, K)).astype(np.int32)
    zeros = rng.integers(0, 16, (G, N)).astype(np.int32)
    scales = rng.uniform(0.005, 0.02, (G, N)).astype(np.float16)
    xs = rng.uniform(0.01, 1, M).astype(np.float32)
    return xq, codes, zeros, scales, xs


@pytest.mark.parametrize("M,N,K", [(1, 16, 128), (5, 32, 256), (17, 48, 384)])
def test_partials_match_bruteforce(M, N, K):
    rng = np.random.default_rng(M * 100 + N)
    xq, codes, zeros, _, _ = _rand_case(rng, M, N, K)
    P = gemm.group_partials(xq, codes, zeros)
    B = gemm.group_partials_bruteforce(xq, codes, zeros)
    np.testing.assert_array_equal(P.astype(np.int64), B)


def test_partials_extremes_fit_int32_exactly():
    K, N = 256, 16
    xq = np.full((2, K), -128, np.int8)
    xq[1] = 127
    codes = np.full((N, K), 15, np.int32)
    zeros = np.zeros((2, N), np.int32)
    P = gemm.group_partials(xq, codes, zeros)
    assert P[0, 0, 0] == -128 * 15 * 128 and P[1, 1, 5] == 127 * 15 * 128
    zeros[:] = 15
    codes[:] = 0
    P = gemm.group_partials(xq, codes, zeros)
    assert P[0, 0, 0] == 128 * 15 * 128


def test_linear_matches_dequant_awq_matmul():
    rng = np.random.default_rng(7)
    M, N, K = 9, 64, 512
    xq, codes, zeros, scales, xs = _rand_case(rng, M, N, K)
    bias = rng.standard_normal(N).astype(np.float32)
    y = gemm.w4a8_linear(xq, xs, codes, scales, zeros, bias)
    W = gemm.dequant_awq(codes, zeros, scales)                     # [N, K]
    ref = (xq.astype(np.float64) * xs[:, None]) @ W.T + bias[None, :]
    np.testing.assert_allclose(y, ref, rtol=1e-12, atol=1e-9)
    # a dropped zero point or transposed scale must be visible
    bad = gemm.w4a8_linear(xq, xs, codes, scales, np.zeros_like(zeros), bias)
    assert np.linalg.norm(bad - ref) / np.linalg.norm(ref) > 0.1


def test_wqlinear_and_awq_dequant_agree():
    """WQLinear stores scaled_zeros = -s*z (qmodule.py:199-203): q*s + sz == (q - z)*s."""
    rng = np.random.default_rng(8)
    N, K = 32, 256
    _, codes, zeros, scales, _ = _rand_case(rng, 1, N, K)
    s = scales.astype(np.float64)
    sz = -(s * zeros)
    np.testing.assert_allclose(gemm.dequant_wqlinear(codes, s, sz), gemm.dequant_awq(codes, zeros, s),
                               rtol=0, atol=1e-12)
