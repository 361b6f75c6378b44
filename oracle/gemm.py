"""Oracle: int4-weight x int8-activation group-scaled GEMM (numpy, CPU).

Restates the Marlin W4A8 computation the reference reaches through
``apply_awq_marlin_linear(..., input_dtype=torch.int8)``
(src/alpamayo_r1/utils/quantization/paroquant_marlin_w4a8.py:314-333) with
AWQ weight semantics ``w = (q - z) * s`` (dequant_awq, 227-235):

  P[m, g, n] = sum_{k in group g} (q[n, k] - z[g, n]) * xq[m, k]      (int32)
  y[m, n]    = xscale[m] * sum_g s[g, n] * P[m, g, n]  (+ bias[n])

Every partial is an integer of magnitude <= 128*15*127 < 2^24, so a float32
matmul over one group is exact regardless of summation order (every
intermediate sum is an integer below 2^24); the partials are exact, and the
epilogue runs in float64.

Marlin additionally recodes the fp16 group scales as int16 plus a global
factor (marlin_act_int8_process_scales, paroquant_marlin_w4a8.py:296-302);
that recoding is vLLM-internal and parity unpinned, so the oracle keeps the
exact fp16 scales (the difference is below 1e-3 relative).
"""

from __future__ import annotations

import numpy as np


def group_partials(xq: np.ndarray, codes_nk: np.ndarray, zeros_gn: np.ndarray,
                   group_size: int = 128) -> np.ndarray:
    """Exact per-group int32 partials P [M, G, N]."""
    xq = np.asarray(xq)
    M, K = xq.shape
    N = codes_nk.shape[0]
    G = K // group_size
    xg = xq.astype(np.float64).reshape(M, G, group_size).transpose(1, 0, 2)          # [G, M, gs]
    w = codes_nk.astype(np.float64).reshape(N, G, group_size) - np.asarray(zeros_gn, np.float64).T[:, :, None]
    wg = w.transpose(1, 2, 0)                                                          # [G, gs, N]
    P = np.matmul(xg, wg)                                                              # [G, M, N]
    return np.ascontiguousarray(P.transpose(1, 0, 2)).astype(np.int32)


def group_partials_bruteforce(xq, codes_nk, zeros_gn, group_size: int = 128) -> np.ndarray:
    """int64 loop form of group_partials (independent check for small shapes)."""
    xq = np.asarray(xq).astype(np.int64)
    M, K = xq.shape
    N = codes_nk.shape[0]
    G = K // group_size
    out = np.zeros((M, G, N), dtype=np.int64)
    q = np.asarray(codes_nk).astype(np.int64)
    z = np.asarray(zeros_gn).astype(np.int64)
    for g in range(G):
        ks = slice(g * group_size, (g + 1) * group_size)
        for n in range(N):
            out[:, g, n] = (xq[:, ks] * (q[n, ks] - z[g, n])[None, :]).sum(axis=1)
    return out


def w4a8_linear(xq: np.ndarray, xscale: np.ndarray, codes_nk: np.ndarray, scales_gn: np.ndarray,
                zeros_gn: np.ndarray, bias: np.ndarray | None = None, group_size: int = 128) -> np.ndarray:
    """float64 output of the W4A8 GEMM (before the final dtype cast)."""
    xq = np.asarray(xq)
    M, K = xq.shape
    N = codes_nk.shape[0]
    G = K // group_size
    s = np.asarray(scales_gn).astype(np.float64)
    z = np.asarray(zeros_gn).astype(np.float32)
    xf = xq.astype(np.float32)
    w = np.asarray(codes_nk).astype(np.float32).reshape(N, G, group_size) - z.T[:, :, None]   # q - z, exact
    acc = np.zeros((M, N), dtype=np.float64)
    for g in range(G):
        P = xf[:, g * group_size:(g + 1) * group_size] @ w[:, g, :].T      # exact integers (< 2^24)
        acc += P.astype(np.float64) * s[g][None, :]
    y = acc * np.asarray(xscale, np.float64)[:, None]
    if bias is not None:
        y = y + np.asarray(bias, np.float64)[None, :]
    return y


def dequant_awq(codes_nk, zeros_gn, scales_gn, group_size: int = 128) -> np.ndarray:
    """w[n, k] = (q - z) * s  (paroquant_marlin_w4a8.py:227-235), float64 [N, K]."""
    q = np.asarray(codes_nk).astype(np.float64)
    z = np.repeat(np.asarray(zeros_gn, np.float64), group_size, axis=0).T
    s = np.repeat(np.asarray(scales_gn).astype(np.float64), group_size, axis=0).T
    return (q - z) * s


def dequant_wqlinear(codes_nk, scales_gn, scaled_zeros_gn, group_size: int = 128) -> np.ndarray:
    """w = q * s + sz  (paroquant_marlin_w4a8.py:216-224), float64 [N, K]."""
    q = np.asarray(codes_nk).astype(np.float64)
    s = np.repeat(np.asarray(scales_gn).astype(np.float64), group_size, axis=0).T
    sz = np.repeat(np.asarray(scaled_zeros_gn).astype(np.float64), group_size, axis=0).T
    return q * s + sz
