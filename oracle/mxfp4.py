"""Oracle: OCP MXFP4 quantization of rotated activations -- TEST INFRASTRUCTURE ONLY.

The reference's fused rotation::rotate_and_quant (kernels/paroquant_kernels/
src/rotation.cu:62-111, 230-315) rotates a float32 tile and quantizes it to
NVFP4.  Its CDNA4 counterpart here quantizes the same float32 rotation result
to MXFP4 as defined by the OCP Microscaling Formats (MX) Specification v1.0:

  * blocks of 32 consecutive elements of a row share one E8M0 scale 2^e
    (byte e + 127; 0xFF is NaN);
  * elements are FP4 E2M1 (sign, 2 exponent bits with bias 1, 1 mantissa
    bit): magnitudes 0, 0.5, 1, 1.5, 2, 3, 4, 6;
  * conversion (spec section 6.3): e = floor(log2(max_i |v_i|)) - 2, where 2
    is the largest exponent of E2M1; each v_i / 2^e is rounded to the nearest
    E2M1 value, ties to the even code, values beyond 6 saturate to 6.

Choices the spec leaves open, fixed here: a block whose absmax is 0 or
subnormal gets e = -127 (the smallest E8M0 scale); a block holding a NaN gets
scale 0xFF and its NaN elements code 0; a block whose absmax is Inf gets e = 126 and its elements
saturate; the sign of zero is kept; element 2i of a row sits in the low
nibble of byte i.

Pinning (tests/test_oracle_mxfp4.py): the E2M1 grid against the bit-level
definition of the format, the E8M0 bytes against torch.float8_e8m0fnu, the
rounding against an exhaustive nearest-value search with explicit ties, and
the round trip of every representable block value.
"""

from __future__ import annotations

import numpy as np

BLOCK = 32
E2M1_GRID = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def shared_exp(amax: np.ndarray) -> np.ndarray:
    """Block exponent e from float32 block absmax values (see the module docstring)."""
    a = np.asarray(amax, np.float32)
    bits = a.view(np.uint32)
    ef = ((bits >> 23) & 0xFF).astype(np.int64)          # biased exponent field
    e = np.where(ef == 0, -127, ef - 127 - 2)              # zero / subnormal -> below the clamp
    return np.maximum(e, -127)


def e2m1_code(y: np.ndarray) -> np.ndarray:
    """E2M1 code (sign << 3 | magnitude index) of y: nearest grid value, ties to the even index."""
    y = np.asarray(y, np.float32)
    a = np.abs(y).astype(np.float64)
    d = np.abs(a[..., None] - E2M1_GRID)                     # distances to the 8 magnitudes
    lo = np.argmin(d, axis=-1)                               # first (lower) index among equal distances
    nxt = np.minimum(lo + 1, 7)
    dl = np.take_along_axis(d, lo[..., None], -1)[..., 0]
    dn = np.take_along_axis(d, nxt[..., None], -1)[..., 0]
    tie = (nxt != lo) & (dl == dn)
    idx = np.where(tie & (lo % 2 == 1), nxt, lo)
    idx = np.where(a > 6, 7, idx)                            # saturation (also +-Inf)
    idx = np.where(np.isnan(a), 0, idx)
    sign = np.signbit(y) & ~np.isnan(y)
    return (idx | (sign.astype(np.int64) << 3)).astype(np.uint8)


def quantize(v: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """float32 [..., H] -> (codes uint8 [..., H/2], scales uint8 [..., H/32])."""
    v = np.asarray(v, np.float32)
    h = v.shape[-1]
    assert h % BLOCK == 0
    blocks = v.reshape(*v.shape[:-1], h // BLOCK, BLOCK)
    with np.errstate(invalid="ignore"):
        amax = np.nanmax(np.abs(blocks), axis=-1) if blocks.size else np.zeros(blocks.shape[:-1], np.float32)
    amax = np.where(np.isnan(amax), np.float32(0), amax).astype(np.float32)   # all-NaN block
    has_nan = np.isnan(blocks).any(axis=-1)
    e = shared_exp(amax)
    scaled = blocks.astype(np.float64) * np.exp2(-e.astype(np.float64))[..., None]   # exact powers of two
    codes = e2m1_code(scaled.astype(np.float32)).reshape(*v.shape[:-1], h)
    packed = (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)
    scales = np.where(has_nan, 255, e + 127).astype(np.uint8)
    return packed, scales


def decode_e2m1(codes: np.ndarray) -> np.ndarray:
    codes = np.asarray(codes, np.int64)
    mag = E2M1_GRID[codes & 7]
    return np.where(codes & 8, -mag, mag)


def dequantize(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """(codes, scales) -> float64 values (NaN for a 0xFF scale)."""
    packed = np.asarray(packed, np.uint8)
    codes = np.stack([packed & 15, packed >> 4], axis=-1).reshape(*packed.shape[:-1], packed.shape[-1] * 2)
    vals = decode_e2m1(codes)
    s = np.asarray(scales, np.int64)
    mult = np.where(s == 255, np.nan, np.exp2(s - 127.0))
    h = codes.shape[-1]
    return (vals.reshape(*vals.shape[:-1], h // BLOCK, BLOCK) * mult[..., None]).reshape(vals.shape)
