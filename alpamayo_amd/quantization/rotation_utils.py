"""Offline rotation utilities (weights / calibration), pure torch.

Mirrors src/alpamayo_r1/utils/quantization/rotation_utils.py:
``apply_rotation_step`` (8-29, the same Givens convention as the kernel),
``rotate_tensor`` (32-77, which *divides* by the channel scales by default so
that W' x' = W x) and ``quantizer`` (80-97).  These run when a checkpoint is
built from an fp model; the inference path uses the HIP kernels.  Unlike the
reference, ``rotate_tensor`` stays on the tensor's own device instead of
forcing ``.cuda()``.
"""

from __future__ import annotations

import torch

from .qmodule import WQLinear
from .quantization_utils import pseudo_quantize_tensor

__all__ = ["apply_rotation_step", "rotate_tensor", "quantizer"]


def apply_rotation_step(t: torch.Tensor, idx_ij: torch.Tensor, theta: torch.Tensor, group_size: int):
    """One Givens layer on rows of t: (xi, xj) <- (c xi + s xj, -s xi + c xj) for every pair."""
    t = t.reshape(-1, t.size(-1)).clone()
    hidden = t.size(-1)
    ng = hidden // group_size
    s = torch.sin(theta).reshape(-1).to(t.dtype)
    c = torch.cos(theta).reshape(-1).to(t.dtype)
    idx = idx_ij.to(torch.int64).reshape(ng, group_size)
    base = (torch.arange(ng, device=idx.device) * group_size)[:, None]
    di = (idx[:, 0::2] + base).reshape(-1)
    dj = (idx[:, 1::2] + base).reshape(-1)
    a = t[:, di]
    b = t[:, dj]
    t[:, di] = c * a + s * b
    t[:, dj] = -s * a + c * b
    return t


def rotate_tensor(tensor, rotation_angles, rotation_pairs, channel_scales, permu=None, divide_scale=True):
    if tensor is None:
        return tensor
    assert rotation_pairs is None or tensor.size(-1) == rotation_pairs.size(-1)
    assert rotation_angles is None or tensor.size(-1) // 2 == rotation_angles.size(-1)
    assert tensor.size(-1) == channel_scales.size(-1)
    assert permu is None or tensor.size(-1) == permu.size(-1)
    shape, dtype, dev = tensor.shape, tensor.dtype, tensor.device
    t = tensor.float().reshape(-1, tensor.size(-1))
    if permu is not None:
        t = t.index_select(-1, permu.to(dev, torch.int64))
    if channel_scales is not None:
        cs = channel_scales.to(dev, torch.float32)
        t = t / cs if divide_scale else t * cs
    if rotation_pairs is not None and rotation_angles is not None:
        pairs = rotation_pairs.to(dev)
        ang = rotation_angles.to(dev, torch.float32)
        for i in range(pairs.size(0)):
            t = apply_rotation_step(t, pairs[i], ang[i], 128)
    return t.to(dtype).reshape(shape)


@torch.no_grad()
def quantizer(linear, w_bit, q_grpsize, qscales=None, qzeros=None):
    """nn.Linear -> WQLinear with (given or computed) per-group scales/zeros."""
    orig = linear.weight.data.detach().clone()
    assert (qscales is None) == (qzeros is None)
    if qscales is None:
        wq, qscales, qzeros = pseudo_quantize_tensor(linear.weight.data, n_bit=w_bit, get_scale_zp=True,
                                                     q_group_size=q_grpsize)
        linear.weight.copy_(wq)
    q = WQLinear.from_linear(linear, w_bit, q_grpsize, False, qscales, qzeros)
    linear.weight.copy_(orig)
    return q
