"""Rotation and RotateLinearInt4 modules.

Mirrors src/alpamayo_r1/utils/quantization/rotation_linear.py:7-139: same
constructor arguments, same persistent buffers (``theta`` [KROT, K/2],
``pairs`` int16 [KROT, K] with group-local indices, ``channel_scales``
[1, K]) and the same ``forward``: ``torch.ops.rotation.rotate(x, pairs,
theta, channel_scales, 128)``.

On top of that, ``Rotation.prepare()`` derives the operands of the fused
rotate+quant kernels (non-persistent, so state-dict keys are unchanged):
  rot_idx    int32 [K/128, 64, 4]     per lane: the channels it starts and
                                      ends with and, per layer, the lane it
                                      fetches its next channel from (validated
                                      as one perfect matching per group and layer)
  rot_cs     float32 [K/128, 64, 8, 2] cos/sin of each pair's angle, evaluated
                                      in float64 on the host and rounded once
  scales_f32 float32 [K]              channel scales
and ``RotateLinearInt4.forward`` runs rotation + int8 quant + GEMM through
``paroquant::w4a8_linear`` when its qlinear is a ``MarlinW4A8Linear``, and
rotation + W4A16 GEMM through ``paroquant::w4a16_linear`` when it is a
``WQLinear``.
"""

from __future__ import annotations

import torch
import torch.nn as nn

from .qmodule import WQLinear
from .quantization_utils import pseudo_quantize_tensor
from .rotation_utils import quantizer, rotate_tensor

__all__ = ["Rotation", "RotateLinearInt4", "check_rotation_pairs"]


def _default_device() -> torch.device:
    return torch.device("cuda") if torch.cuda.is_available() else torch.device("cpu")


def check_rotation_pairs(pairs: torch.Tensor, group_size: int = 128) -> None:
    """Raise ValueError unless each layer pairs every channel of each group exactly once."""
    p = pairs.detach().to("cpu", torch.int64)
    krot, h = p.shape
    if h % group_size:
        raise ValueError(f"dim {h} is not a multiple of group_size {group_size}")
    if p.numel() and (p.min() < 0 or p.max() >= group_size):
        raise ValueError("rotation pairs must be group-local indices in [0, group_size)")
    s = torch.sort(p.view(krot, h // group_size, group_size), dim=-1).values
    if not torch.equal(s, torch.arange(group_size).expand_as(s)):
        raise ValueError("every rotation layer must pair each channel of a group exactly once")


class Rotation(nn.Module):
    def __init__(self, dim, krot=8, group_size=128, rotation_angles=None, rotation_pairs=None, channel_scales=None):
        super().__init__()
        if krot != 8 or group_size != 128:
            raise NotImplementedError()
        assert dim % group_size == 0
        num_groups = dim // group_size
        device = _default_device()
        if rotation_angles is None:
            rotation_angles = torch.zeros(krot, dim // 2, device=device, dtype=torch.float16)
        if rotation_pairs is None:
            single = torch.randperm(group_size, dtype=torch.int, device=device)
            rotation_pairs = single.repeat(num_groups).unsqueeze(0).expand(krot, -1)
        if channel_scales is None:
            channel_scales = torch.ones(1, dim, dtype=torch.half)
        self.register_buffer("theta", rotation_angles.clone().contiguous())
        self.register_buffer("pairs", rotation_pairs.clone().short().contiguous())
        self.register_buffer("channel_scales", channel_scales.clone().contiguous())
        self.register_buffer("rot_idx", torch.empty(0, dtype=torch.int32), persistent=False)
        self.register_buffer("rot_cs", torch.empty(0, dtype=torch.float32), persistent=False)
        self.register_buffer("scales_f32", torch.empty(0, dtype=torch.float32), persistent=False)
        self.group_size = group_size
        self._prep_src = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return torch.ops.rotation.rotate(x, self.pairs, self.theta, self.channel_scales, 128)

    @torch.no_grad()
    def prepare(self) -> None:
        """(Re)derive the fused kernel's operands from theta/pairs/channel_scales (host work: call it before
        graph capture; the forward paths call it when ``prepared`` is False) and register them for
        rotation::rotate on these buffers."""
        from ..ops import pack_rotation, register_packed_rotation

        dev = self.theta.device
        check_rotation_pairs(self.pairs, self.group_size)
        rot_idx, rot_cs = pack_rotation(self.pairs, self.cos_sin_table())
        self.rot_idx = rot_idx.to(dev)
        self.rot_cs = rot_cs.to(dev)
        self.scales_f32 = self.channel_scales.detach().reshape(-1).to(dev, torch.float32).contiguous()
        self._prep_src = self._param_source()
        register_packed_rotation(self.pairs, self.theta, self.channel_scales, self.rot_idx, self.rot_cs,
                                 self.scales_f32)

    def _param_source(self):
        from ..ops import tensor_state

        return tuple(tensor_state(t) for t in (self.theta, self.pairs, self.channel_scales))

    def cos_sin_table(self) -> torch.Tensor:
        """float32 [KROT, K/2, 2] (cos, sin) of theta, evaluated in float64 on the host."""
        th = self.theta.detach().to("cpu").float().double()
        return torch.stack([torch.cos(th), torch.sin(th)], dim=-1).float()

    @property
    def krot(self) -> int:
        return self.pairs.size(0)

    @property
    def prepared(self) -> bool:
        """True while the packed operands were derived from the current theta / pairs / channel_scales:
        False again after load_state_dict, an in-place update or a move of any of them.  Buffers created under
        torch.inference_mode() carry no version counter, so only a replacement or a move of them is seen:
        after changing such a buffer in place, call prepare()."""
        return self.rot_cs.numel() > 0 and self._prep_src == self._param_source()


class RotateLinearInt4(nn.Module):
    def __init__(self, in_feat, out_feat, bias, dtype, rotation_angles=None, rotation_pairs=None,
                 channel_scales=None):
        super().__init__()
        self.in_features = in_feat
        self.out_features = out_feat
        self.rotation = Rotation(in_feat, rotation_angles=rotation_angles, rotation_pairs=rotation_pairs,
                                 channel_scales=channel_scales)
        self.qlinear = WQLinear(4, 128, self.in_features, self.out_features, bias, dtype=dtype)

    @classmethod
    def from_linear(cls, linear, rotation_angles=None, rotation_pairs=None, channel_scales=None, qscales=None,
                    qzeros=None, rotate_weight=False, init_only=True):
        """Offline construction from an nn.Linear (rotation_linear.py:68-118)."""
        rl = cls(linear.in_features, linear.out_features, linear.bias is not None, linear.weight.dtype,
                 rotation_angles, rotation_pairs, channel_scales)
        if rotate_weight:
            with torch.no_grad():
                w = linear.weight.data.detach().clone()
                w = rotate_tensor(w, rotation_angles, rotation_pairs, channel_scales)
                if qscales is not None:
                    w = pseudo_quantize_tensor(w, 4, q_group_size=128, qzeros=qzeros, qscales=qscales)
                    qzeros = qzeros.view(w.size(0), -1)
                    qscales = qscales.view(w.size(0), -1)
                linear.weight.copy_(w)
        if init_only:
            return rl
        linear.to(torch.half)
        assert (qscales is None) == (qzeros is None)
        rl.qlinear = quantizer(linear, 4, 128, qscales=qscales, qzeros=qzeros)
        return rl

    @torch.no_grad()
    def forward(self, x):
        from .paroquant_marlin_w4a8 import MarlinW4A8Linear

        if isinstance(self.qlinear, MarlinW4A8Linear):
            # rotation (fp16 result) -> per-token int8 -> W4A8 GEMM, fused.
            return self.qlinear.forward_rotated(x, self.rotation, input_fp16=False, out_dtype=x.dtype)
        if isinstance(self.qlinear, WQLinear):
            # rotation (fp16 result) -> W4A16 GEMM behind one entry point.
            q, rot = self.qlinear, self.rotation
            if not torch.compiler.is_compiling():
                if not q.prepared:
                    q.prepare()
                if not rot.prepared:
                    rot.prepare()
            return torch.ops.paroquant.w4a16_linear(x, rot.rot_idx, rot.rot_cs, rot.scales_f32, rot.krot, q.w16_pack,
                                                    q.w16_meta, q.bias, False, x.dtype)
        x = self.rotation(x)
        return self.qlinear(x)

    def buffer_name(self, buffer_name: str):
        table = {
            "qlinear.qweight": lambda: self.qlinear.qweight,
            "qlinear.scaled_zeros": lambda: self.qlinear.scaled_zeros,
            "qlinear.scales": lambda: self.qlinear.scales,
            "rotation.theta": lambda: self.rotation.theta,
            "rotation.pairs": lambda: self.rotation.pairs,
            "rotation.channel_scales": lambda: self.rotation.channel_scales,
        }
        if buffer_name not in table:
            raise ValueError(f"Invalid buffer name: {buffer_name}")
        return table[buffer_name]()
