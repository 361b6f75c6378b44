"""Autograd wrapper of rotation::rotate.

Mirrors kernels/paroquant_kernels/interface.py:6-96 (``RotateTensorFunc`` and
``scaled_pairwise_rotation``).  The backward inverts the rotation one layer at
a time with rotate(., idx[i], -theta[i]) in reverse layer order
(interface.py:42-50), gathers the pair values to form
d theta = sum_rows(g_i b - g_j a) cos - sum_rows(g_i a + g_j b) sin
(interface.py:55-76) and d scale = sum_rows(x * g) (84-87).
"""

from __future__ import annotations

import torch


class RotateTensorFunc(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, idx_ij, theta, scale=None, group_size=128):
        ctx.orig_shape, ctx.orig_dtype = x.shape, x.dtype
        ctx.has_scale = scale is not None
        ctx.group_size = group_size
        y = torch.ops.rotation.rotate(x, idx_ij, theta, scale, group_size)
        saved = (x, idx_ij, theta, y) + ((scale,) if ctx.has_scale else ())
        ctx.save_for_backward(*saved)
        return y

    @staticmethod
    def backward(ctx, grad_out):
        saved = list(ctx.saved_tensors)
        x, idx_ij, theta, y = saved[:4]
        scale = saved[4] if ctx.has_scale else None
        gs = ctx.group_size
        H = x.size(-1)
        g = grad_out.reshape(-1, H).contiguous()
        krot = idx_ij.size(0)
        ng = H // gs
        B = y.numel() // H
        t = y.reshape(B, H)
        grad_theta = torch.zeros_like(theta)
        offs = (torch.arange(ng, device=idx_ij.device, dtype=torch.int64) * gs).unsqueeze(1)
        for i in range(krot - 1, -1, -1):
            th_neg = (-theta[i:i + 1]).contiguous()
            idx_i = idx_ij[i:i + 1].contiguous()
            t_prev = torch.ops.rotation.rotate(t, idx_i, th_neg, None, gs)
            g_prev = torch.ops.rotation.rotate(g, idx_i, th_neg, None, gs)
            chunk = idx_i.reshape(ng, gs).to(torch.int64)
            di = (chunk[:, 0::2] + offs).reshape(-1)
            dj = (chunk[:, 1::2] + offs).reshape(-1)
            a = t_prev[:, di].reshape(B, ng, gs // 2)
            b = t_prev[:, dj].reshape(B, ng, gs // 2)
            ga = g[:, di].reshape(B, ng, gs // 2)
            gb = g[:, dj].reshape(B, ng, gs // 2)
            grad_s = (ga * b - gb * a).sum(dim=0)
            grad_c = (ga * a + gb * b).sum(dim=0)
            th = theta[i].reshape(ng, gs // 2)
            grad_theta[i] = (grad_s * th.cos() - grad_c * th.sin()).reshape(-1).to(theta.dtype)
            t, g = t_prev, g_prev
        if ctx.has_scale:
            grad_x = g * scale.reshape(1, H)
            grad_scale = (x.reshape(B, H) * g).sum(dim=0).to(scale.dtype).reshape(scale.shape)
        else:
            grad_x, grad_scale = g, None
        return grad_x.reshape(ctx.orig_shape).to(ctx.orig_dtype), None, grad_theta, grad_scale, None


def scaled_pairwise_rotation(x, idx_ij, theta, scales=None, group_size=128):
    return RotateTensorFunc.apply(x, idx_ij, theta, scales, group_size)
