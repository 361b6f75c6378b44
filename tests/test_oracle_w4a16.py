"""Pins the W4A16 oracle (oracle/w4a16.py) on the CPU.

The weights w16 = fp16(q * s + sz) are checked against a library routine
(torch's fp16 addcmul, one rounding of the float32 value), against the AWQ
convention (q - z) * s when sz = -s * z is representable, and the GEMM against
a loop that forms and rounds every weight on its own."""

import numpy as np
import pytest
import torch

from oracle import gemm as ogemm
from oracle import w4a16 as ow

RNG = np.random.default_rng(1604)


def _weights(n, k, rng=RNG, exact_zero=False):
    g = k // 128
    codes = rng.integers(0, 16, size=(n, k), dtype=np.int64)
    zeros = rng.integers(0, 16, size=(g, n), dtype=np.int64)
    if exact_zero:
        # 7 significant bits: s * z (<= 11 bits) and (q - z) * s are exact in fp16
        scales = (rng.integers(64, 128, size=(g, n)) * 2.0 ** rng.integers(-16, -8, size=(g, n))).astype(np.float16)
    else:
        scales = rng.uniform(0.002, 0.03, size=(g, n)).astype(np.float16)
    sz = (-(scales.astype(np.float32) * zeros.astype(np.float32))).astype(np.float16)
    return codes, scales, sz, zeros


def test_w16_is_fp16_addcmul_of_the_checkpoint_values():
    codes, scales, sz, _ = _weights(48, 384)
    w16 = ow.dequant_w16(codes, scales, sz)
    s = torch.from_numpy(np.repeat(scales, 128, axis=0).T.copy())
    z = torch.from_numpy(np.repeat(sz, 128, axis=0).T.copy())
    q = torch.from_numpy(codes.astype(np.float16))
    ref = torch.addcmul(z, q, s).numpy()          # fp16 in, one rounding of the float32 value
    assert np.array_equal(w16.view(np.uint16), ref.view(np.uint16))


def test_w16_formula_is_exact_before_its_one_rounding():
    codes, scales, sz, _ = _weights(32, 256)
    # the reference's dequant_wqlinear evaluates q * s + sz in float32; that value is exact
    q32 = codes.astype(np.float32)
    s32 = np.repeat(scales.astype(np.float32), 128, axis=0).T
    z32 = np.repeat(sz.astype(np.float32), 128, axis=0).T
    v32 = q32 * s32 + z32
    assert np.array_equal(v32.astype(np.float64), ogemm.dequant_wqlinear(codes, scales, sz))
    assert np.array_equal(v32.astype(np.float16), ow.dequant_w16(codes, scales, sz))


def test_w16_equals_awq_semantics_when_zero_is_representable():
    codes, scales, sz, zeros = _weights(32, 256, exact_zero=True)
    assert np.array_equal(sz.astype(np.float64), -(scales.astype(np.float64) * zeros))   # sz = -s*z exactly
    w16 = ow.dequant_w16(codes, scales, sz).astype(np.float64)
    assert np.array_equal(w16, ogemm.dequant_awq(codes, zeros, scales))


@pytest.mark.parametrize("m,n,k,with_bias", [(1, 16, 128, False), (3, 32, 256, True), (9, 16, 384, True)])
def test_gemm_matches_bruteforce(m, n, k, with_bias):
    codes, scales, sz, _ = _weights(n, k)
    x = RNG.standard_normal((m, k)).astype(np.float16)
    bias = RNG.standard_normal(n).astype(np.float16) if with_bias else None
    y = ow.w4a16_gemm(x, codes, scales, sz, bias)
    yb = ow.w4a16_gemm_bruteforce(x, codes, scales, sz, bias)
    np.testing.assert_allclose(y, yb, rtol=1e-12, atol=1e-12)


def test_gemm_close_to_unrounded_weights():
    # one fp16 rounding of each weight moves y by at most 2^-11 relative per term
    codes, scales, sz, _ = _weights(64, 512)
    x = RNG.standard_normal((5, 512)).astype(np.float16)
    y16 = ow.w4a16_gemm(x, codes, scales, sz)
    yex = x.astype(np.float64) @ ogemm.dequant_wqlinear(codes, scales, sz).T
    bound = np.abs(x.astype(np.float64)) @ np.abs(ogemm.dequant_wqlinear(codes, scales, sz)).T * 2.0 ** -11
    assert np.all(np.abs(y16 - yex) <= bound + 1e-12)
