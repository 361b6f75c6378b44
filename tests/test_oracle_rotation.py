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


def _dense_autograd_grads(x, pairs, theta, scales, gy, gs):
    """dL/d(x, theta, scales) of L = sum(gy * y) by torch float64 autograd through an explicit dense product
    of block-diagonal Givens matrices built from (pairs, theta) with torch.cos / torch.sin."""
    import torch

    krot, h = pairs.shape
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    tt = torch.tensor(theta.astype(np.float32).astype(np.float64), requires_grad=True)
    st = torch.tensor(scales.astype(np.float64), requires_grad=True) if scales is not None else None
    v = xt * st if st is not None else xt
    for r in range(krot):
        rows_i, cols_i, vals = [], [], []
        L = torch.zeros(h, h, dtype=torch.float64)
        for g in range(h // gs):
            for t in range(gs // 2):
                i = g * gs + int(pairs[r, g * gs + 2 * t])
                j = g * gs + int(pairs[r, g * gs + 2 * t + 1])
                a = tt[r, g * gs // 2 + t]
                L = L.index_put((torch.tensor([i, i, j, j]), torch.tensor([i, j, i, j])),
                                torch.stack([torch.cos(a), torch.sin(a), -torch.sin(a), torch.cos(a)]))
        v = v @ L.T
    (v * torch.tensor(gy, dtype=torch.float64)).sum().backward()
    return xt.grad.numpy(), tt.grad.numpy(), (st.grad.numpy() if st is not None else None)


@pytest.mark.parametrize("gs,krot,scaled", [(128, 8, True), (64, 4, True), (128, 2, False), (128, 16, True)])
def test_backward_matches_float64_autograd(gs, krot, scaled):
    """rotate_backward against autograd of the dense product (a library routine over a different form)."""
    rng = np.random.default_rng(10 + krot)
    h, rows = 128 if gs == 128 else 192, 5
    pairs = _random_pairs(rng, krot, h, gs)
    theta = rng.uniform(-np.pi, np.pi, (krot, h // 2)).astype(np.float16)
    scales = rng.uniform(0.5, 2, h).astype(np.float16) if scaled else None
    x = rng.standard_normal((rows, h))
    gy = rng.standard_normal((rows, h))
    gx, gt, gsc = rotation.rotate_backward(x, pairs, theta, scales, gy, gs)
    rx, rt, rs = _dense_autograd_grads(x, pairs, theta, scales, gy, gs)
    # the oracle uses cos/sin rounded to float32, autograd exact ones: agreement to ~1e-7
    assert np.linalg.norm(gx - rx) / np.linalg.norm(rx) < 1e-6
    assert np.linalg.norm(gt - rt) / np.linalg.norm(rt) < 1e-6
    if scaled:
        assert np.linalg.norm(gsc - rs) / np.linalg.norm(rs) < 1e-6
    else:
        assert gsc is None


def test_backward_angle_gradient_by_finite_differences():
    """d L / d theta[r, p] by central differences of the forward oracle (float64 angles)."""
    rng = np.random.default_rng(21)
    h, krot, rows = 128, 3, 4
    pairs = _random_pairs(rng, krot, h)
    theta = rng.uniform(-np.pi, np.pi, (krot, h // 2)).astype(np.float32)
    x = rng.standard_normal((rows, h))
    gy = rng.standard_normal((rows, h))
    _, gt, _ = rotation.rotate_backward(x, pairs, theta, None, gy, 128)
    gi, gj = rotation.pair_index_arrays(pairs, 128)

    def loss(th):
        t = x.copy()
        for r in range(krot):
            c, s = np.cos(th[r]), np.sin(th[r])
            a, b = t[:, gi[r]], t[:, gj[r]]
            t[:, gi[r]], t[:, gj[r]] = c * a + s * b, c * b - s * a
        return float((t * gy).sum())

    eps = 1e-6
    th64 = theta.astype(np.float64)
    for r, p in ((0, 0), (1, 17), (2, 63)):
        tp, tm = th64.copy(), th64.copy()
        tp[r, p] += eps
        tm[r, p] -= eps
        fd = (loss(tp) - loss(tm)) / (2 * eps)
        assert abs(fd - gt[r, p]) < 1e-5 * max(1.0, abs(fd)), (r, p, fd, gt[r, p])


def test_backward_check_catches_a_sign_mistake():
    """A plausible mistake in the angle gradient (g_a' a' + g_b' b' instead of g_a' b' - g_b' a') must fail the
    autograd comparison above."""
    rng = np.random.default_rng(22)
    h, krot, rows = 128, 2, 3
    pairs = _random_pairs(rng, krot, h)
    theta = rng.uniform(-np.pi, np.pi, (krot, h // 2)).astype(np.float16)
    x = rng.standard_normal((rows, h))
    gy = rng.standard_normal((rows, h))
    _, rt, _ = _dense_autograd_grads(x, pairs, theta, None, gy, 128)
    # wrong form, planted on the CPU
    c32, s32 = rotation.cos_sin_table(theta)
    gi, gj = rotation.pair_index_arrays(pairs, 128)
    t = x.copy()
    outs = []
    for r in range(krot):
        a, b = t[:, gi[r]], t[:, gj[r]]
        na, nb = c32[r] * a + s32[r] * b, c32[r] * b - s32[r] * a
        t[:, gi[r]], t[:, gj[r]] = na, nb
        outs.append((na, nb))
    g = gy.copy()
    wrong = np.zeros((krot, h // 2))
    for r in range(krot - 1, -1, -1):
        na, nb = outs[r]
        ga, gb = g[:, gi[r]], g[:, gj[r]]
        wrong[r] = (ga * na + gb * nb).sum(axis=0)
        g[:, gi[r]], g[:, gj[r]] = c32[r] * ga - s32[r] * gb, s32[r] * ga + c32[r] * gb
    assert np.linalg.norm(wrong - rt) / np.linalg.norm(rt) > 0.1
