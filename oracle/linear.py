"""Oracle: one ParoQuant W4A8 linear end to end (numpy, CPU).

Follows the reference call chain of §3.2 in the module docs:
``BF16RotateLinearWrapper.forward`` (paroquant_marlin_w4a8.py:59-65) casts the
bf16 activations to fp16, ``RotateLinearInt4.forward`` (rotation_linear.py:
120-124) rotates them with ``torch.ops.rotation.rotate`` (fp16 in, fp16
out), ``MarlinW4A8Linear.forward`` (paroquant_marlin_w4a8.py:314-333)
quantizes per token to int8 and runs the int4 x int8 GEMM, and the wrapper
casts the result back to bf16.

numpy has no bfloat16, so bf16 tensors are carried as float32 arrays whose
values are exactly representable in bf16 (see ``bf16_round``).
"""

from __future__ import annotations

import numpy as np

from . import gemm, quant, rotation


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (round-to-nearest-even), returned as float32."""
    f = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    b = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    rounded = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    out = rounded.astype(np.uint32).view(np.float32).copy()
    out[nan] = np.nan
    return out


def bf16_bits(x_bf16_as_f32: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(x_bf16_as_f32, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def rotate_quant(x_bf16_as_f32, pairs, cos, sin, scales_f32, group_size=128,
                 input_fp16=True, materialize_fp16=True):
    """Fused stage 1+2: returns (rotated float32 [M, K], codes int8 [M, K], scale float32 [M])."""
    v = rotation.rotate_path_f32(x_bf16_as_f32, pairs, cos, sin, scales_f32, group_size,
                                 input_fp16=input_fp16, materialize_fp16=materialize_fp16)
    q, s = quant.quant_int8_per_token(v)
    return v, q, s


def w4a8_rotate_linear(x_bf16_as_f32, pairs, cos, sin, scales_f32, codes_nk, wscales_gn, zeros_gn,
                       bias=None, group_size=128, input_fp16=True, materialize_fp16=True):
    """Whole linear. Returns (y float64 [M, N] before the output cast, codes, xscale)."""
    _, q, s = rotate_quant(x_bf16_as_f32, pairs, cos, sin, scales_f32, group_size,
                           input_fp16, materialize_fp16)
    y = gemm.w4a8_linear(q, s, codes_nk, wscales_gn, zeros_gn, bias, group_size)
    return y, q, s


def reference_path_dequant(x_bf16_as_f32, pairs, cos, sin, scales_f32, awq_qweight, awq_scales,
                           awq_qzeros, bias=None, group_size=128):
    """The reference path as a CPU user would run it, from the AWQ buffers.

    Unpacks the AWQ int32 weights every call, dequantizes them
    (dequant_awq), multiplies the dequantized int8 activations in float32 and
    rounds the result to bf16.  This is the timed CPU baseline.
    """
    v = rotation.rotate_path_f32(x_bf16_as_f32, pairs, cos, sin, scales_f32, group_size)
    q, s = quant.quant_int8_per_token(v)
    K = awq_qweight.shape[0]
    N = awq_qweight.shape[1] * 8
    codes_kn = _unpack_awq_f32(awq_qweight, N)                          # [K, N]
    zeros = _unpack_awq_f32(awq_qzeros, N)                              # [G, N]
    sc = np.asarray(awq_scales).astype(np.float32)                      # [G, N]
    G = K // group_size
    w = (codes_kn.reshape(G, group_size, N) - zeros[:, None, :]) * sc[:, None, :]
    y = (q.astype(np.float32) @ w.reshape(K, N)) * s[:, None]
    if bias is not None:
        y = y + np.asarray(bias, np.float32)[None, :]
    return bf16_round(y)


def _unpack_awq_f32(packed: np.ndarray, cols: int) -> np.ndarray:
    p = np.asarray(packed).view(np.uint32)
    rows = p.shape[0]
    out = np.empty((rows, cols // 8, 8), dtype=np.float32)
    for i, dst in enumerate(_AWQ_ORDER):
        out[:, :, dst] = (p >> np.uint32(4 * i)) & np.uint32(0xF)
    return out.reshape(rows, cols)


from .packing import AWQ_ORDER as _AWQ_ORDER  # noqa: E402
