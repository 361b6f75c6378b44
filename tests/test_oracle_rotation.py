"""Pins oracle/rotation.py against closed forms, invariants and brute force.

Reference semantics: kernels/paroquant_kernels/src/rotation.cuh:247-337 and
rotation_utils.py:8-29 (xi' = c xi + s xj, xj' = -s xi + c xj on the pair
(idx[2t], idx[2t+1]) of each group, channel scale multiplied first).
"""

import math

import numpy as np
import pytest

from oracle import rotation


def _random_pairs(rng, krot, h, gs=128):
    return np.concatenate([np.stack([rng.permutation(gs) for _ in range(h // gs)]).reshape(-1)[None]
                           for _ in range(krot)]).astype(np.int16)


def _dense_matrix(pairs, theta, gs):
    """Explicit float64 product R_{K-1} ... R_0 (each R_r block-diagonal Givens)."""
    krot, h = pairs.shape
    R = np.eye(h)
    th = theta.astype(np.float32).astype(np.float64)
    for r in range(krot):
        L = np.eye(h)
        for g in range(h // gs):
            for t in range(gs // 2):
                i = g * gs + int(pairs[r, g * gs + 2 * t])
                j = g * gs + int(pairs[r, g * gs + 2 * t + 1])
                c, s = math.cos(th[r, g * gs // 2 + t]), math.sin(th[r, g * gs // 2 + t])
                L[i, i], L[i, j] = c, s
                L[j, i], L[j, j] = -s, c
        R = L @ R
    return R


@pytest.mark.parametrize("gs,krot", [(128, 8), (64, 4), (128, 1), (128, 16)])
def test_closed_form_dense_product(gs, krot):
    rng = np.random.default_rng(1)
    h = 256
    pairs = _random_pairs(rng, krot, h, gs)
    theta = rng.uniform(-np.pi, np.pi, (krot, h // 2)).astype(np.float16)
    scales = rng.uniform(0.5, 2, h).astype(np.float16)
    x = rng.standard_normal((5, h)).astype(np.float32)
    y = rotation.rotate(x, pairs, theta, scales, gs, out_dtype=np.float32)
    R = _dense_matrix(pairs, theta, gs)
    ref = (x.astype(np.float64) * scales.astype(np.float64)) @ R.T
    err = np.linalg.norm(y - ref) / np.linalg.norm(ref)
    assert err < 1e-6, err


def test_closed_form_catches_sign_and_index_mistakes():
    """The closed-form check must reject a plausible wrong oracle (flipped sign / swapped pair)."""
    rng = np.random.default_rng(2)
    h, gs, krot = 128, 128, 2
    pairs = _random_pairs(rng, krot, h)
    theta = rng.uniform(-np.pi, np.pi, (krot, h // 2)).astype(np.float16)
    x = rng.standard_normal((3, h)).astype(np.float32)
    R = _dense_matrix(pairs, theta, gs)
    ref = x.astype(np.float64) @ R.T
    good = rotation.rotate(x, pairs, theta, None, gs, out_dtype=np.float32)
    assert np.linalg.norm(good - ref) / np.linalg.norm(ref) < 1e-6
    bad_sign = rotation.rotate(x, pairs, -theta, None, gs, out_dtype=np.float32)
    swapped = pairs.copy()
    swapped[:, 0::2], swapped[:, 1::2] = pairs[:, 1::2], pairs[:, 0::2]
    bad_idx = rotation.rotate(x, swapped, theta, None, gs, out_dtype=np.float32)
    for bad in (bad_sign, bad_idx):
        assert np.linalg.norm(bad - ref) / np.linalg.norm(ref) > 1e-2


def test_norm_preserved_per_group_without_scales():
    rng = np.random.default_rng(3)
    h, gs = 512, 128
    pairs = _random_pairs(rng, 8, h)
    theta = rng.uniform(-np.pi, np.pi, (8, h // 2)).astype(np.float16)
    x = (rng.standard_normal((7, h)) * 3).astype(np.float32)
    y = rotation.rotate(x, pairs, theta, None, gs, out_dtype=np.float32)
    nx = np.linalg.norm(x.reshape(7, -1, gs), axis=-1)
    ny = np.linalg.norm(y.reshape(7, -1, gs), axis=-1)
    np.testing.assert_allclose(ny, nx, rtol=1e-5)


def test_inverse_layers_with_negative_angles_is_identity():
    """The reference backward (interface.py:42-50) undoes layer i with rotate(., idx[i], -theta[i])."""
    rng = np.random.default_rng(4)
    h, gs, krot = 256, 128, 8
    pairs = _random_pairs(rng, krot, h)
    theta = rng.uniform(-np.pi, np.pi, (krot, h // 2)).astype(np.float32)
    x = rng.standard_normal((4, h)).astype(np.float32)
    y = rotation.rotate(x, pairs, theta, None, gs, out_dtype=np.float32)
    for r in range(krot - 1, -1, -1):
        y = rotation.rotate(y, pairs[r:r + 1], -theta[r:r + 1], None, gs, out_dtype=np.float32)
    np.testing.assert_allclose(y, x, atol=2e-5)


def test_theta_zero_is_scale_only_and_half_pi_swaps():
    rng = np.random.default_rng(5)
    h, gs = 128, 128
    pairs = _random_pairs(rng, 1, h)
    x = rng.standard_normal((2, h)).astype(np.float32)
    s = rng.uniform(0.5, 2, h).astype(np.float16)
    y0 = rotation.rotate(x, pairs, np.zeros((1, h // 2), np.float16), s, gs, out_dtype=np.float32)
    np.testing.assert_array_equal(y0, (x * s.astype(np.float32)).astype(np.float32))
    y1 = rotation.rotate(x, pairs, np.full((1, h // 2), np.pi / 2, np.float32), None, gs, out_dtype=np.float32)
    i, j = pairs[0, 0::2].astype(int), pairs[0, 1::2].astype(int)
    np.testing.assert_allclose(y1[:, i], x[:, j], atol=1e-6)
    np.testing.assert_allclose(y1[:, j], -x[:, i], atol=1e-6)


def test_brute_force_loop_matches_vectorized_bit_exactly():
    """Per-pair Python loop transcribing rotation.cuh:299-314 (fp32 with the fma form)."""
    rng = np.random.default_rng(6)
    h, gs, krot = 128, 128, 8
    pairs = _random_pairs(rng, krot, h)
    theta = rng.uniform(-np.pi, np.pi, (krot, h // 2)).astype(np.float16)
    sc = rng.uniform(0.5, 2, h).astype(np.float16)
    x = rng.standard_normal((2, h)).astype(np.float16)
    vec = rotation.rotate(x, pairs, theta, sc, gs, out_dtype=np.float32)
    c, s = rotation.cos_sin_table(theta)
    for row in range(2):
        buf = [np.float32(np.float32(x[row, k]) * np.float32(sc[k])) for k in range(h)]
        for r in range(krot):
            for t in range(gs // 2):
                i, j = int(pairs[r, 2 * t]), int(pairs[r, 2 * t + 1])
                xi, xj = buf[i], buf[j]
                cc, ss = c[r, t], s[r, t]
                buf[i] = np.float32(float(xi) * float(cc) + float(np.float32(xj * ss)))
                buf[j] = np.float32(float(xj) * float(cc) - float(np.float32(xi * ss)))
        np.testing.assert_array_equal(np.array(buf, np.float32), vec[row])


def test_leading_dims_and_dtype_round_trip():
    rng = np.random.default_rng(7)
    h = 256
    pairs = _random_pairs(rng, 8, h)
    theta = rng.uniform(-np.pi, np.pi, (8, h // 2)).astype(np.float16)
    x = rng.standard_normal((2, 3, h)).astype(np.float16)
    y = rotation.rotate(x, pairs, theta, None, 128)
    assert y.shape == x.shape and y.dtype == np.float16
    flat = rotation.rotate(x.reshape(6, h), pairs, theta, None, 128)
    np.testing.assert_array_equal(y.reshape(6, h), flat)


def test_check_pairs_rejects_non_matchings():
    rng = np.random.default_rng(8)
    p = _random_pairs(rng, 2, 256)
    rotation.check_pairs(p, 128)
    bad = p.copy()
    bad[1, 5] = bad[1, 6]
    with pytest.raises(ValueError):
        rotation.check_pairs(bad, 128)
    with pytest.raises(ValueError):
        rotation.check_pairs(p.astype(np.int64) + 1, 128)


def test_rotate_rejects_bad_shapes():
    with pytest.raises(ValueError):
        rotation.rotate(np.zeros((1, 100), np.float32), np.zeros((8, 100), np.int16),
                        np.zeros((8, 50), np.float32), None, 128)
    with pytest.raises(ValueError):
        rotation.rotate(np.zeros((1, 128), np.float32), np.zeros((8, 128), np.int16),
                        np.zeros((4, 64), np.float32), None, 128)
