"""WQLinear checkpoint module and its int16 weight packing.

Mirrors src/alpamayo_r1/utils/quantization/qmodule.py: the same buffer
names, shapes and dtypes (``qweight`` int16 [N/4, K], ``scales`` and
``scaled_zeros`` [calculate_zeros_width(K)*8, N], optional ``bias``), so
ParoQuant state dicts load unchanged.

``WQLinear.forward`` is the reference's W4A16 path (qmodule.py:207-232),
there the un-vendored ``torch.ops.awq.gemv`` / ``gemm`` kernels; here
``paroquant::w4a16_gemm``: fp16 activations times the weights
fp16(q * scales + scaled_zeros) (one rounding), float32 accumulation, plus
bias.  ``prepare()`` derives the kernel's packed weights (non-persistent
buffers ``w16_pack`` / ``w16_meta``, so state-dict keys are unchanged); the
first forward after the checkpoint buffers change re-derives them (call
``prepare()`` ahead of a graph capture).
"""

from __future__ import annotations

import torch
import torch.nn as nn

__all__ = ["make_divisible", "calculate_zeros_width", "pack_intweight", "unpack_intweight", "WQLinear"]


def make_divisible(c: int, divisor: int) -> int:
    return (c + divisor - 1) // divisor


def calculate_zeros_width(in_features: int, group_size: int = 128, pack_num: int = 8) -> int:
    """Rows/8 of the scales buffers (qmodule.py:24-36)."""
    if group_size >= 128:
        mult = 1
    elif group_size == 64:
        mult = 2
    elif group_size == 32:
        mult = 4
    else:
        raise NotImplementedError
    base = make_divisible(in_features // group_size, pack_num)
    return make_divisible(base, mult) * mult


def _k_source(K: int, device) -> torch.Tensor:
    """Original K index held at each packed position: inside each 32-block,
    position 8a + 4c + b holds 8b + 2a + c (the two K shuffles of qmodule.py:45-55)."""
    p = torch.arange(32, device=device)
    a, rem = p // 8, p % 8
    c, b = rem // 4, rem % 4
    src = 8 * b + 2 * a + c
    return (torch.arange(K // 32, device=device)[:, None] * 32 + src[None, :]).reshape(K)


def pack_intweight(unpacked_qweight: torch.Tensor, interleave: int = 4, kstride: int = 64) -> torch.Tensor:
    """int4 codes [N, K] -> WQLinear int16 [N/4, K] (qmodule.py:39-78)."""
    w = unpacked_qweight.to(torch.int32)
    N, K = w.shape
    w = w[:, _k_source(K, w.device)]
    nb = N // interleave
    w = w.reshape(nb, interleave, K // kstride, kstride).permute(0, 2, 1, 3).reshape(nb, K // kstride, kstride, interleave)
    packed = torch.zeros((nb, K // kstride, kstride), dtype=torch.int32, device=w.device)
    for f in range(interleave):
        packed |= (w[..., f] & 0xF) << (4 * f)
    packed = torch.where(packed >= 32768, packed - 65536, packed)
    return packed.reshape(nb, K).to(torch.int16).contiguous()


def unpack_intweight(qweight: torch.Tensor, out_features: int, in_features: int,
                     interleave: int = 4, kstride: int = 64) -> torch.Tensor:
    """WQLinear int16 [N/4, K] -> int4 codes [N, K] int32 (inverse of pack_intweight)."""
    N, K = out_features, in_features
    pw = qweight.contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
    pw = pw.reshape(N // interleave, K // kstride, kstride)
    nib = torch.stack([(pw >> (4 * f)) & 0xF for f in range(interleave)], dim=-1)
    tiles = nib.reshape(N // interleave, K // kstride, interleave, kstride).permute(0, 2, 1, 3)
    shuffled = tiles.reshape(N, K)
    out = torch.empty_like(shuffled)
    out[:, _k_source(K, shuffled.device)] = shuffled
    return out


class WQLinear(nn.Module):
    """ParoQuant / AWQ W4 checkpoint container (qmodule.py:91-243)."""

    def __init__(self, w_bit, group_size, in_features, out_features, bias, dtype=torch.float16):
        super().__init__()
        if w_bit not in [4]:
            raise NotImplementedError("Only 4-bit are supported for now.")
        self.in_features = in_features
        self.out_features = out_features
        self.w_bit = w_bit
        self.group_size = group_size if group_size != -1 else in_features
        self.split_k_iters = 8
        self.interleave = 4
        assert self.in_features % self.group_size == 0
        assert out_features % (32 // self.w_bit) == 0
        pack_num = 32 // self.w_bit
        int16_pack_num = 16 // self.w_bit
        assert out_features % self.interleave == 0
        zw = calculate_zeros_width(in_features, self.group_size) * pack_num
        self.register_buffer("qweight", torch.zeros(
            (out_features // self.interleave, in_features // int16_pack_num * self.interleave), dtype=torch.int16))
        self.register_buffer("scales", torch.zeros((zw, out_features), dtype=dtype))
        self.register_buffer("scaled_zeros", torch.zeros((zw, out_features), dtype=dtype))
        if bias:
            self.register_buffer("bias", torch.zeros((out_features), dtype=dtype))
        else:
            self.bias = None
        self.register_buffer("w16_pack", torch.empty(0, dtype=torch.uint8), persistent=False)
        self.register_buffer("w16_meta", torch.empty(0, dtype=torch.int32), persistent=False)
        self._w16_src = None

    @classmethod
    def from_linear(cls, linear, w_bit, group_size, init_only=False, scales=None, zeros=None):
        """Quantize an nn.Linear with given per-group scales/zeros [N, K/G] (qmodule.py:149-205)."""
        q = cls(w_bit, group_size, linear.in_features, linear.out_features, linear.bias is not None,
                dtype=linear.weight.data.dtype)
        if init_only:
            return q
        assert scales is not None and zeros is not None
        dtype = scales.dtype
        pack_num = 32 // q.w_bit
        zw = calculate_zeros_width(linear.in_features, group_size) * pack_num
        qscales = torch.zeros((scales.shape[0], zw), dtype=dtype, device=scales.device)
        qscales[:, : scales.shape[1]] = scales
        q.scales = qscales.transpose(1, 0).contiguous()
        if linear.bias is not None:
            q.bias = linear.bias.clone().to(dtype)
        scale_zeros = zeros * scales
        gidx = torch.arange(linear.in_features, device=scales.device) // group_size
        w = linear.weight.data
        intweight = torch.round((w + scale_zeros[:, gidx].to(w.dtype)) / qscales[:, gidx].to(w.dtype)).to(torch.int32)
        q.qweight = pack_intweight(intweight.contiguous(), interleave=4, kstride=64)
        scaled_zeros = torch.zeros_like(qscales)
        scaled_zeros[:, : scales.shape[1]] = -(qscales[:, : scales.shape[1]] * zeros.to(torch.float32)).to(dtype)
        q.scaled_zeros = scaled_zeros.transpose(1, 0).contiguous()
        return q

    def _w16_source(self):
        from ..ops import tensor_state

        return tuple(tensor_state(t) for t in (self.qweight, self.scales, self.scaled_zeros))

    @property
    def prepared(self) -> bool:
        return self.w16_pack.numel() > 0 and self._w16_src == self._w16_source()

    @torch.no_grad()
    def prepare(self) -> None:
        """(Re)derive the W4A16 kernel's packed weights from qweight / scales / scaled_zeros."""
        from .paroquant_marlin_w4a8 import pack_awq_int32

        if self.group_size != 128:
            raise NotImplementedError(f"the W4A16 kernels take group_size 128, not {self.group_size}")
        n, k = self.out_features, self.in_features
        g = k // self.group_size
        codes = unpack_intweight(self.qweight, n, k)
        awq = pack_awq_int32(codes.t().contiguous())
        self.w16_pack, self.w16_meta = torch.ops.paroquant.w4a16_prepack(
            awq, self.scales[:g].to(torch.float16).contiguous(), self.scaled_zeros[:g].to(torch.float16).contiguous())
        self._w16_src = self._w16_source()

    @torch.no_grad()
    def forward(self, inputs):
        """inputs: fp16 [..., K] -> fp16 [..., N] (qmodule.py:207-232)."""
        if not torch.compiler.is_compiling() and not self.prepared:
            self.prepare()
        return torch.ops.paroquant.w4a16_gemm(inputs, self.w16_pack, self.w16_meta, self.bias, inputs.dtype)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, bias={self.bias is not None}, "
                f"w_bit={self.w_bit}, group_size={self.group_size}")
