"""Autograd wrapper of rotation::rotate.

The reference exposes ``RotateTensorFunc`` and ``scaled_pairwise_rotation``
(kernels/paroquant_kernels/interface.py:6-96) with these names and
arguments.  Forward is ``rotation::rotate``; backward is one call of
``paroquant::rotate_backward`` (a single HIP kernel pass plus a fixed-order
reduction), which recomputes the layers from x and returns the gradients
for x, theta and the channel scales.  The gradient formulas are in
alpamayo_amd/csrc/pq_rotate_bwd.hip.
"""

from __future__ import annotations

import torch


class RotateTensorFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, idx_ij, theta, scale=None, group_size=128):
        ctx.group_size = group_size
        ctx.scaled = scale is not None
        ctx.save_for_backward(x, idx_ij, theta, *((scale,) if ctx.scaled else ()))
        return torch.ops.rotation.rotate(x, idx_ij, theta, scale, group_size)

    @staticmethod
    def backward(ctx, grad_y):
        x, idx_ij, theta, *rest = ctx.saved_tensors
        scale = rest[0] if ctx.scaled else None
        grad_x, grad_theta, grad_scale = torch.ops.paroquant.rotate_backward(
            grad_y.to(x.dtype).contiguous(), x, idx_ij, theta, scale, ctx.group_size)
        return grad_x, None, grad_theta, (grad_scale if ctx.scaled else None), None


def scaled_pairwise_rotation(x, idx_ij, theta, scales=None, group_size=128):
    return RotateTensorFunc.apply(x, idx_ij, theta, scales, group_size)
