"""Elementwise steps of a decoder layer in front of its W4A8 linears -- TEST INFRASTRUCTURE ONLY.

RMSNorm (below), the residual add (``residual_sum``) and the gated MLP's
activation (``swiglu``).

Restates Qwen3VLTextRMSNorm.forward
(src/alpamayo_r1/models/qwen3_vl/modeling_qwen3_vl.py:354-359) with the
residual add a decoder layer makes before it (``residual + hidden_states``
in the activation dtype):

  s = x + residual, rounded to the activation dtype (s = x without residual)
  v = s in float32;  var = mean(v^2) in float32;  r = rsqrt(var + eps)
  h = weight * (v * r rounded to the activation dtype), rounded to the dtype

The reference computes var with torch's float32 reduction and rsqrt in
float32; here var is the float64 mean of the float32 squares rounded to
float32 and r = 1 / sqrt(var + eps) rounded once to float32.  The two can
differ in the last bit of r, which moves h only where v * r lies within an
ulp of a rounding boundary of the activation dtype (tests allow 1 ulp).

Arrays carry bf16 / fp16 values as float32 (exactly representable values).
"""

from __future__ import annotations

import numpy as np

from .linear import bf16_round


def round_to(v: np.ndarray, dtype: str) -> np.ndarray:
    v = np.asarray(v, dtype=np.float32)
    if dtype == "bf16":
        return bf16_round(v)
    if dtype == "f16":
        return v.astype(np.float16).astype(np.float32)
    return v


def residual_sum(x: np.ndarray, residual: np.ndarray | None, dtype: str) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    if residual is None:
        return x
    return round_to(x + np.asarray(residual, dtype=np.float32), dtype)


def rms_factor(s: np.ndarray, eps: float) -> np.ndarray:
    """Per-row rsqrt(mean(s^2) + eps) as float32 ([..., k] -> [..., 1])."""
    v = np.asarray(s, dtype=np.float32)
    sq = (v * v).astype(np.float64)
    var = np.float32(1.0) * (sq.sum(axis=-1, keepdims=True) / v.shape[-1]).astype(np.float32)
    t = (var + np.float32(eps)).astype(np.float32)
    return (1.0 / np.sqrt(t.astype(np.float64))).astype(np.float32)


def rmsnorm(x: np.ndarray, weight: np.ndarray, eps: float, residual: np.ndarray | None = None,
            dtype: str = "bf16") -> tuple[np.ndarray, np.ndarray]:
    """(h, s): the normalized rows and the residual sum, both in `dtype` (as float32)."""
    s = residual_sum(x, residual, dtype)
    r = rms_factor(s, eps)
    w = np.asarray(weight, dtype=np.float32)
    h = round_to(w * round_to(s * r, dtype), dtype)
    return h, s


def swiglu(gate: np.ndarray, up: np.ndarray, dtype: str = "bf16") -> np.ndarray:
    """A gated MLP's down_proj input, act_fn(gate_proj(x)) * up_proj(x) with SiLU
    (patches.py:541-548), in the module's rounding: silu in float32
    (g / (1 + exp(-g))) rounded to `dtype`, times up, rounded to `dtype`."""
    g = np.asarray(gate, dtype=np.float32)
    with np.errstate(over="ignore"):
        a = round_to(g / (np.float32(1) + np.exp(-g)), dtype)
    return round_to(a * np.asarray(up, dtype=np.float32), dtype)
