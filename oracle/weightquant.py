"""Oracle: offline asymmetric uint4 weight quantizer (numpy, CPU).

Restates ``pseudo_quantize_tensor`` (src/alpamayo_r1/utils/quantization/
quantization_utils.py:18-73) for the zero-point branch ParoQuant uses, per
``q_group_size`` group of each row:

  s = clamp(max - min, min=1e-5) / 15
  z = clamp(-round(min / s), 0, 15)
  q = clamp(round(w / s) + z, 0, 15)
  w_hat = (q - z) * s

``round`` is round-half-to-even (torch.round).  Arithmetic is float32 like
the reference's float32 tensors.
"""

from __future__ import annotations

import numpy as np


def pseudo_quantize(w: np.ndarray, n_bit: int = 4, q_group_size: int = 128):
    """Returns (w_hat float32 [N, K], codes int32 [N, K], scales float32 [N, G], zeros float32 [N, G])."""
    w = np.asarray(w, dtype=np.float32)
    N, K = w.shape
    wg = w.reshape(-1, q_group_size)
    max_int = np.float32(2 ** n_bit - 1)
    mx = wg.max(axis=1, keepdims=True)
    mn = wg.min(axis=1, keepdims=True)
    s = (np.maximum(mx - mn, np.float32(1e-5)) / max_int).astype(np.float32)
    z = np.clip(-np.rint((mn / s).astype(np.float32)), 0, max_int).astype(np.float32)
    q = np.clip(np.rint((wg / s).astype(np.float32)) + z, 0, max_int).astype(np.float32)
    w_hat = ((q - z) * s).astype(np.float32)
    G = K // q_group_size
    return (w_hat.reshape(N, K), q.reshape(N, K).astype(np.int32),
            s.reshape(N, G), z.reshape(N, G))
