"""Pins oracle/quant.py (per-token symmetric int8) by closed form and invariants.

The reference quantizes inside vLLM (paroquant_marlin_w4a8.py:319-333);
vLLM is not available, so the tie-breaking rule is parity unpinned (the bar
allows 1 LSB there).  Everything else is fixed by these checks.
"""

import numpy as np

from oracle import quant


def test_closed_form_and_invariants():
    rng = np.random.default_rng(0)
    v = (rng.standard_normal((64, 512)) * rng.uniform(0.1, 50, (64, 1))).astype(np.float32)
    v[:, 3] *= 20
    q, s = quant.quant_int8_per_token(v)
    absmax = np.abs(v).max(axis=1)
    np.testing.assert_array_equal(s, (absmax / np.float32(127)).astype(np.float32))
    assert q.dtype == np.int8
    assert np.all(np.abs(q).max(axis=1) == 127)            # the absmax element maps to +-127
    assert np.all(np.sign(q[q != 0]) == np.sign(v[q != 0]))  # sign preserved
    err = np.abs(q.astype(np.float64) * s[:, None] - v)
    assert np.all(err <= 0.5 * s[:, None] * (1 + 1e-5))      # round-to-nearest
    # an off-by-one scale (x/absmax*128) or truncation would break one of these
    trunc = np.trunc(v * (np.float32(127) / absmax)[:, None])
    assert np.any(trunc != q)


def test_zero_row_and_spike():
    v = np.zeros((3, 256), np.float32)
    v[1, 17] = -3.5
    v[2] = np.linspace(-1, 1, 256)
    q, s = quant.quant_int8_per_token(v)
    assert s[0] == 0 and np.all(q[0] == 0)
    assert q[1, 17] == -127 and np.count_nonzero(q[1]) == 1
    assert q[2, 0] == -127 and q[2, -1] == 127


def test_round_half_even_on_exact_ties():
    # absmax 127 -> inv 1: x = 2.5 -> 2, 3.5 -> 4, -0.5 -> 0
    v = np.array([[127.0, 2.5, 3.5, -0.5, 0.5, -1.5]], np.float32)
    q, s = quant.quant_int8_per_token(v)
    np.testing.assert_array_equal(q[0], [127, 2, 4, 0, 0, -2])
    assert s[0] == 1.0
