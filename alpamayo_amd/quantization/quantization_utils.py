"""Offline weight quantization helpers.

Mirrors src/alpamayo_r1/utils/quantization/quantization_utils.py:
``set_op_by_name`` and ``pseudo_quantize_tensor`` (asymmetric uintN per
group: s = clamp(max-min, 1e-5)/(2^n-1), z = clamp(-round(min/s), 0, 2^n-1),
w_hat = (clamp(round(w/s)+z) - z) * s).  Used when building checkpoints, not
on the inference path.
"""

from __future__ import annotations

import torch

__all__ = ["set_op_by_name", "pseudo_quantize_tensor"]


def set_op_by_name(layer, name, new_module):
    levels = name.split(".")
    mod = layer
    for lv in levels[:-1]:
        mod = mod[int(lv)] if lv.isdigit() else getattr(mod, lv)
    setattr(mod, levels[-1], new_module)


def pseudo_quantize_tensor(w, n_bit=8, zero_point=True, q_group_size=-1, inplace=False, get_scale_zp=False,
                           qzeros=None, qscales=None):
    org_shape = w.shape
    if q_group_size > 0:
        assert org_shape[-1] % q_group_size == 0
        w = w.reshape(-1, q_group_size)
    assert w.dim() == 2
    assert (qscales is None) == (qzeros is None)
    max_int = 2 ** n_bit - 1
    min_int = 0
    if qscales is None:
        if not zero_point:
            raise NotImplementedError("only the zero-point branch is used by ParoQuant")
        max_val = w.amax(dim=1, keepdim=True)
        min_val = w.amin(dim=1, keepdim=True)
        qscales = (max_val - min_val).clamp(min=1e-5) / max_int
        qzeros = (-torch.round(min_val / qscales)).clamp_(min_int, max_int)
    else:
        qscales = qscales.reshape(-1, 1)
        qzeros = qzeros.reshape(-1, 1)
    assert torch.isnan(qscales).sum() == 0
    assert torch.isnan(w).sum() == 0
    if inplace:
        w.div_(qscales).round_().add_(qzeros).clamp_(min_int, max_int).sub_(qzeros).mul_(qscales)
    else:
        w = (torch.clamp(torch.round(w / qscales) + qzeros, min_int, max_int) - qzeros) * qscales
    assert torch.isnan(w).sum() == 0
    w = w.reshape(org_shape)
    if get_scale_zp:
        return w, qscales.view(w.shape[0], -1), qzeros.view(w.shape[0], -1)
    return w
