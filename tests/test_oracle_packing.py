"""Pins oracle/packing.py and oracle/weightquant.py.

  * pack_intweight / calculate_zeros_width / pseudo_quantize_tensor: golden
    vectors written by the reference's own functions (tests/golden/make_golden.py);
  * AWQ order [0, 2, 4, 6, 1, 3, 5, 7] (paroquant_marlin_w4a8.py:149): a
    hand-derived known-answer vector;
  * every inverse by round trip; the kernel layout by explicit element checks.
"""

import numpy as np
import pytest

from oracle import packing, weightquant


@pytest.mark.parametrize("tag", ["a", "b", "c"])
def test_pack_intweight_golden(golden, tag):
    codes = golden[f"pack_{tag}_codes"]
    expect = golden[f"pack_{tag}_packed"]
    np.testing.assert_array_equal(packing.pack_intweight(codes), expect)
    np.testing.assert_array_equal(packing.unpack_wqlinear_qweight(expect, *codes.shape), codes)


def test_calculate_zeros_width_golden(golden):
    for k, gs, zw in golden["zeros_width_table"]:
        assert packing.calculate_zeros_width(int(k), int(gs)) == zw


@pytest.mark.parametrize("tag", ["a", "b"])
def test_pseudo_quantize_golden(golden, tag):
    w = golden[f"pq_{tag}_w"]
    w_hat, codes, s, z = weightquant.pseudo_quantize(w)
    np.testing.assert_array_equal(w_hat, golden[f"pq_{tag}_what"])
    np.testing.assert_array_equal(s, golden[f"pq_{tag}_scales"])
    np.testing.assert_array_equal(z, golden[f"pq_{tag}_zeros"])
    assert codes.min() >= 0 and codes.max() <= 15


def test_awq_known_answer():
    vals = np.arange(8, dtype=np.int32)[None, :]            # columns 0..7 hold values 0..7
    packed = packing.pack_awq_int32(vals)
    # nibble i holds column AWQ_ORDER[i] = 0,2,4,6,1,3,5,7
    assert packed.view(np.uint32)[0, 0] == 0x75316420
    np.testing.assert_array_equal(packing.unpack_awq_int32(packed, 8), vals)


def test_awq_round_trip_and_wqlinear_to_awq():
    rng = np.random.default_rng(0)
    N, K = 64, 512
    G = K // 128
    codes = rng.integers(0, 16, (N, K)).astype(np.int32)
    zeros = rng.integers(0, 16, (G, N)).astype(np.int32)
    scales = rng.uniform(0.005, 0.02, (G, N)).astype(np.float16)
    q16 = packing.pack_intweight(codes)
    zw = packing.calculate_zeros_width(K) * 8
    sc_full = np.zeros((zw, N), np.float16)
    sc_full[:G] = scales
    sz_full = np.zeros((zw, N), np.float16)
    sz_full[:G] = (-(scales.astype(np.float32) * zeros)).astype(np.float16)
    awq_qw, awq_sc, awq_qz, c2, z2 = packing.wqlinear_to_awq(q16, sc_full, sz_full, N, K, 128)
    np.testing.assert_array_equal(c2, codes)
    np.testing.assert_array_equal(z2, zeros)
    np.testing.assert_array_equal(packing.unpack_awq_int32(awq_qw, N), codes.T)
    np.testing.assert_array_equal(packing.unpack_awq_int32(awq_qz, N), zeros)
    np.testing.assert_array_equal(awq_sc, scales)


def test_kernel_layout_round_trip_and_elements():
    rng = np.random.default_rng(1)
    N, K = 48, 384
    G = K // 128
    codes = rng.integers(0, 16, (N, K)).astype(np.int32)
    zeros = rng.integers(0, 16, (G, N)).astype(np.int32)
    scales = rng.uniform(0.005, 0.02, (G, N)).astype(np.float16)
    wpack, wmeta = packing.prepack_kernel_layout(codes, scales, zeros)
    assert wpack.shape == (N // 16, G, 64, 16) and wmeta.shape == (N // 16, G, 16)
    c2, s2, z2 = packing.unpack_kernel_layout(wpack, wmeta)
    np.testing.assert_array_equal(c2, codes)
    np.testing.assert_array_equal(s2, scales)
    np.testing.assert_array_equal(z2, zeros)
    # spot-check the documented byte formula
    for (n, k) in [(0, 0), (17, 200), (47, 383), (5, 131)]:
        tile, c, g = n // 16, n % 16, k // 128
        j, d, rem = (k % 128) // 32, (k % 32) // 8, k % 8
        i, nib = rem % 4, rem // 4
        byte = wpack[tile, g, 16 * j + c, 4 * d + i]
        assert (byte >> (4 * nib)) & 0xF == codes[n, k]
    meta = wmeta[2, 1, 3]   # n = 35, g = 1
    assert (meta >> 16) == zeros[1, 35]
    assert np.uint16(meta & 0xFFFF).view(np.float16) == scales[1, 35]
