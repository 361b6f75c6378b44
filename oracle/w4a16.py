"""Oracle: the W4A16 linear (WQLinear.forward) -- TEST INFRASTRUCTURE ONLY.

WQLinear.forward (src/alpamayo_r1/utils/quantization/qmodule.py:207-232)
multiplies fp16 activations by the int4 weights through
``torch.ops.awq.gemv`` (fewer than 8 rows) or ``torch.ops.awq.gemm``, from
the un-vendored ParoQuant ``inference_engine`` (absent here, no pinned
version), then adds the bias.  The weight semantics are those of
``dequant_wqlinear`` (paroquant_marlin_w4a8.py:216-224): w = q * s + sz with
the fp16 ``scales`` s and ``scaled_zeros`` sz of the (group, column).  Those
kernels form the weights in fp16 before multiplying; the oracle rounds the
exact value of q * s + sz once to fp16 (q * s + sz is exact in float64: a
4-bit integer times an 11-bit significand plus an fp16 value):

  w16[n, k] = fp16(q[n, k] * s[g, n] + sz[g, n])
  y[m, n]   = sum_k x[m, k] * w16[n, k]  (+ bias[n])      in float64

The rotated variant (RotateLinearInt4.forward, rotation_linear.py:136-139)
rounds the rotation's result to fp16 first (rotation::rotate on fp16
activations returns fp16).

Pinning (tests/test_oracle_w4a16.py): w16 against the reference's own
dequant formula evaluated in float32 as it does (exact there, then one fp16
rounding); with sz = -s * z representable, w16 equals dequant_awq's
(q - z) * s exactly; the GEMM against an int64/float64 brute-force loop on
small shapes.  How the external kernels round inside their accumulation is
parity unpinned (they are not in the reference tree); the bar for the HIP
kernels is float32 accumulation of the exact products of x and w16.
"""

from __future__ import annotations

import numpy as np

from . import rotation


def dequant_w16(codes_nk, scales_gn, scaled_zeros_gn, group_size: int = 128) -> np.ndarray:
    """float16 [N, K]: fp16(q * s + sz), one rounding of the exact value."""
    q = np.asarray(codes_nk).astype(np.float64)
    s = np.repeat(np.asarray(scales_gn, np.float16).astype(np.float64), group_size, axis=0).T
    sz = np.repeat(np.asarray(scaled_zeros_gn, np.float16).astype(np.float64), group_size, axis=0).T
    return (q * s + sz).astype(np.float16)


def w4a16_gemm(x_f16, codes_nk, scales_gn, scaled_zeros_gn, bias=None, group_size: int = 128) -> np.ndarray:
    """float64 [M, N] output (before the output cast)."""
    x = np.asarray(x_f16, np.float16).astype(np.float64)
    w = dequant_w16(codes_nk, scales_gn, scaled_zeros_gn, group_size).astype(np.float64)
    y = x @ w.T
    if bias is not None:
        y = y + np.asarray(bias).astype(np.float64)[None, :]
    return y


def w4a16_gemm_bruteforce(x_f16, codes_nk, scales_gn, scaled_zeros_gn, bias=None, group_size: int = 128):
    """Loop form for small shapes: every weight formed and rounded on its own."""
    x = np.asarray(x_f16, np.float16)
    q = np.asarray(codes_nk)
    s = np.asarray(scales_gn, np.float16)
    sz = np.asarray(scaled_zeros_gn, np.float16)
    M, K = x.shape
    N = q.shape[0]
    y = np.zeros((M, N), dtype=np.float64)
    for n in range(N):
        for k in range(K):
            g = k // group_size
            w = float(np.float16(int(q[n, k]) * float(s[g, n]) + float(sz[g, n])))
            y[:, n] += x[:, k].astype(np.float64) * w
        if bias is not None:
            y[:, n] += float(bias[n])
    return y


def rotate_linear_w16(x, pairs, cos, sin, scales_f32, codes_nk, scales_gn, scaled_zeros_gn, bias=None,
                      group_size: int = 128, input_fp16: bool = False):
    """RotateLinearInt4 with a WQLinear: (y float64 [M, N], rotated fp16 rows)."""
    v = rotation.rotate_path_f32(x, pairs, cos, sin, scales_f32, group_size, input_fp16=input_fp16,
                                 materialize_fp16=True)
    v16 = v.astype(np.float16)
    return w4a16_gemm(v16, codes_nk, scales_gn, scaled_zeros_gn, bias, group_size), v16
