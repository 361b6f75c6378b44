"""Pins the MXFP4 oracle (oracle/mxfp4.py) on the CPU against the OCP MX v1.0
definition: the E2M1 grid from the format's bit fields, E8M0 bytes from
torch.float8_e8m0fnu, round-to-nearest-even at every midpoint, saturation,
round trips and the error bound."""

import numpy as np
import pytest
import torch

from oracle import mxfp4 as mx

RNG = np.random.default_rng(4404)


def test_grid_matches_the_bit_level_definition():
    # E2M1: s | e1 e0 | m ; exponent bias 1; e = 0 is subnormal (0.5 * m)
    for c in range(16):
        s, e, m = c >> 3, (c >> 1) & 3, c & 1
        mag = 0.5 * m if e == 0 else 2.0 ** (e - 1) * (1 + 0.5 * m)
        assert mx.decode_e2m1(np.array([c]))[0] == (-mag if s else mag)


def test_e8m0_bytes_match_torch():
    for k in range(-125, 128):
        block = np.zeros(32, np.float32)
        block[7] = 1.5 * 2.0 ** k                     # floor(log2(amax)) = k
        _, sc = mx.quantize(block[None])
        want = torch.tensor([2.0 ** (k - 2)], dtype=torch.float64).to(torch.float8_e8m0fnu).view(torch.uint8)
        assert int(sc[0, 0]) == int(want[0]) == k - 2 + 127


@pytest.mark.parametrize("y,code", [(0.25, 0), (0.75, 2), (1.25, 2), (1.75, 4), (2.5, 4), (3.5, 6), (5.0, 6),
                                    (0.2, 0), (0.3, 1), (1.0, 2), (5.5, 7), (7.9, 7), (100.0, 7)])
def test_rounding_known_answers(y, code):
    assert mx.e2m1_code(np.float32(y)) == code
    assert mx.e2m1_code(np.float32(-y)) == code | 8


def test_midpoints_round_to_even_and_neighbours_to_nearest():
    g = mx.E2M1_GRID
    for i in range(7):
        mid = np.float32((g[i] + g[i + 1]) / 2)
        even = i if i % 2 == 0 else i + 1
        assert mx.e2m1_code(mid) == even
        assert mx.e2m1_code(np.nextafter(mid, np.float32(0))) == i
        assert mx.e2m1_code(np.nextafter(mid, np.float32(10))) == i + 1


def test_signed_zero_nan_inf_and_zero_blocks():
    assert mx.e2m1_code(np.float32(-0.0)) == 8
    zero = np.zeros((1, 32), np.float32)
    q, s = mx.quantize(zero)
    assert s[0, 0] == 0 and not q.any()
    b = RNG.standard_normal((1, 64)).astype(np.float32)
    b[0, 40] = np.nan
    q, s = mx.quantize(b)
    assert s[0, 0] != 255 and s[0, 1] == 255
    b[0, 40] = np.inf
    q, s = mx.quantize(b)
    assert s[0, 1] == 126 + 127 and (q[0, 20] & 15) == 7
    assert mx.e2m1_code(np.float32(-np.inf)) == 15


def test_round_trip_of_representable_blocks():
    e = RNG.integers(-120, 120, size=(50, 4))
    codes = RNG.integers(0, 16, size=(50, 4, 32))
    codes[:, :, 0] = RNG.integers(6, 8, size=(50, 4))    # amax in [4, 6] * 2^e pins the exponent
    v = (mx.decode_e2m1(codes) * np.exp2(e)[..., None]).reshape(50, 128).astype(np.float32)
    q, s = mx.quantize(v)
    assert np.array_equal(s.astype(np.int64), e + 127)
    assert np.array_equal(mx.dequantize(q, s), v.astype(np.float64))


def test_error_bound():
    v = (RNG.standard_normal((64, 256)) * np.exp2(RNG.integers(-20, 20, size=(64, 1)))).astype(np.float32)
    q, s = mx.quantize(v)
    d = mx.dequantize(q, s)
    scale = np.repeat(np.exp2(s.astype(np.float64) - 127), 32, axis=1)
    y = np.abs(v) / scale
    step = np.where(y < 2, 0.5, np.where(y < 4, 1.0, 2.0))
    err = np.abs(d - v) / scale
    sat = y > 6
    assert np.all(err[~sat] <= step[~sat] / 2 + 1e-12)
    assert np.all(err[sat] < 2.0)
    assert np.all(y < 8)                                  # amax / 2^e is in [4, 8)
