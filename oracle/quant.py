"""Oracle: per-token symmetric int8 activation quantization (numpy, CPU).

The reference quantizes the rotated fp16 activations inside vLLM's
``apply_awq_marlin_linear(..., input_dtype=torch.int8)``
(src/alpamayo_r1/utils/quantization/paroquant_marlin_w4a8.py:319-333), i.e.
vLLM's dynamic per-token ``scaled_int8_quant``.  vLLM is not vendored, not
pinned and not installed, so this restates its published algorithm:

  absmax[m] = max_k |x[m, k]|              (in float32)
  scale[m]  = absmax[m] / 127
  q[m, k]   = saturate_int8(round_half_even(x[m, k] * (127 / absmax[m])))

A row whose absmax is 0 gets scale 0 and codes 0.

Parity: pinned by the closed form and invariants in tests/test_oracle_quant.py;
the tie-breaking rule and the multiply-by-reciprocal form are parity
unpinned (the acceptance bar allows 1 LSB for them).
"""

from __future__ import annotations

import numpy as np


def quant_int8_per_token(v: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Quantize float rows v [rows, h] -> (int8 codes [rows, h], float32 scale [rows])."""
    v = np.asarray(v, dtype=np.float32)
    absmax = np.max(np.abs(v), axis=-1) if v.shape[-1] else np.zeros(v.shape[:-1], np.float32)
    absmax = absmax.astype(np.float32)
    nz = absmax > 0
    inv = np.zeros_like(absmax)
    inv[nz] = (np.float32(127.0) / absmax[nz]).astype(np.float32)
    prod = (v * inv[..., None]).astype(np.float32)
    q = np.clip(np.rint(prod), -128, 127).astype(np.int8)
    scale = (absmax / np.float32(127.0)).astype(np.float32)
    return q, scale


def dequant_int8(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    return q.astype(np.float64) * np.asarray(scale, np.float64)[..., None]
