"""Shared helpers of the GPU parity tests (test infrastructure)."""

from __future__ import annotations

import numpy as np
import torch


def to_np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        t = t.float()
    return t.numpy()


def rel_fro(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    d = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (d if d > 0 else 1.0))


def assert_codes_close(got: np.ndarray, ref: np.ndarray, min_identical=0.999):
    """int8 codes: >= 99.9% identical and never more than 1 LSB apart."""
    diff = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    frac = float(np.mean(diff == 0)) if diff.size else 1.0
    assert diff.max(initial=0) <= 1, f"codes differ by {diff.max()} LSB"
    assert frac >= min_identical, f"only {frac:.6f} of codes identical"
    return frac


def assert_bf16_close(got: np.ndarray, ref64: np.ndarray, tol_fro=1e-2):
    """Final outputs: within 1e-2 relative (Frobenius), and elementwise within
    a few bf16 ulps of the float64 oracle."""
    e = rel_fro(got, ref64)
    assert e <= tol_fro, f"relative Frobenius error {e:.3e}"
    scale = np.sqrt(np.mean(np.asarray(ref64, np.float64) ** 2)) + 1e-30
    bound = 2.0 ** -7 * np.abs(ref64) + 1e-3 * scale
    bad = np.abs(np.asarray(got, np.float64) - ref64) > bound
    assert not bad.any(), f"{bad.sum()} outputs beyond the elementwise bound; e.g. got {got[bad][:4]} ref {ref64[bad][:4]}"
    return e


def packed_rotation(pairs: torch.Tensor, theta: torch.Tensor):
    """(rot_idx, rot_cs, cos, sin) for Rotation-style pairs [krot, K] and angles [krot, K/2]."""
    from alpamayo_amd.ops import pack_rotation
    from oracle import rotation as orot

    c, s = orot.cos_sin_table(theta.numpy())
    cs = torch.from_numpy(np.stack([c, s], axis=-1)).contiguous()
    rot_idx, rot_cs = pack_rotation(pairs.to(torch.int16), cs)
    return rot_idx, rot_cs, c, s
