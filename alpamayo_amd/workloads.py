"""Seeded synthetic inputs of the W4A8 benchmark configurations.

Value distributions (one 8B decoder layer's seven quantized linears):
  activations   bf16 [M, K] ~ N(0, 1), 1% of channels (randperm) scaled x20
  rotation      8 layers; per 128-channel group and layer an independent
                random pairing (randperm -> pairs (p[2t], p[2t+1])), angles
                U(-pi, pi) stored fp16, channel scales U(0.5, 2) fp16
  weights       codes U{0..15}, group scales fp16 U(0.005, 0.02), zero
                points U{6..9}; packed to AWQ int32 (K, N/8) as the
                reference's load_from_awq expects
Shapes: q/o 4096->4096, k/v 4096->1024, gate/up 4096->12288, down 12288->4096.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

KROT = 8
GROUP = 128

# name -> (out_features N, in_features K)
QWEN3_8B_LINEARS = {
    "q_proj": (4096, 4096),
    "k_proj": (1024, 4096),
    "v_proj": (1024, 4096),
    "o_proj": (4096, 4096),
    "gate_proj": (12288, 4096),
    "up_proj": (12288, 4096),
    "down_proj": (4096, 12288),
}

AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


def generator(seed: int, device="cpu") -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def activations(M: int, K: int, gen: torch.Generator, device="cpu", outlier_frac=0.01, outlier_mult=20.0):
    x = torch.randn(M, K, generator=gen, device=device, dtype=torch.float32)
    n_out = int(math.ceil(outlier_frac * K))
    cols = torch.randperm(K, generator=gen, device=device)[:n_out]
    x[:, cols] *= outlier_mult
    return x.to(torch.bfloat16)


def rotation_params(K: int, gen: torch.Generator, device="cpu", krot=KROT):
    """(pairs int16 [krot, K] group-local, theta fp16 [krot, K/2], channel_scales fp16 [1, K])."""
    G = K // GROUP
    keys = torch.rand(krot, G, GROUP, generator=gen, device=device)
    perm = torch.argsort(keys, dim=-1)                       # a random permutation per (layer, group)
    pairs = perm.reshape(krot, K).to(torch.int16)
    theta = ((torch.rand(krot, K // 2, generator=gen, device=device) * 2 - 1) * math.pi).to(torch.float16)
    scales = (0.5 + 1.5 * torch.rand(1, K, generator=gen, device=device)).to(torch.float16)
    return pairs.contiguous(), theta.contiguous(), scales.contiguous()


def pack_awq(values: torch.Tensor) -> torch.Tensor:
    """[rows, cols] int4 -> [rows, cols/8] int32, nibble i = column 8c + AWQ_ORDER[i]."""
    rows, cols = values.shape
    v = values.to(torch.int32).reshape(rows, cols // 8, 8)
    out = torch.zeros(rows, cols // 8, dtype=torch.int32, device=values.device)
    for i, src in enumerate(AWQ_ORDER):
        out |= (v[:, :, src] & 0xF) << (4 * i)
    return out


@dataclass
class Weights:
    awq_qweight: torch.Tensor   # int32 [K, N/8]
    awq_scales: torch.Tensor    # fp16 [G, N]
    awq_qzeros: torch.Tensor    # int32 [G, N/8]
    codes: torch.Tensor | None  # uint8 [N, K] (kept only on request)
    zeros: torch.Tensor         # int32 [G, N]


def weights(N: int, K: int, gen: torch.Generator, device="cpu", keep_codes=False) -> Weights:
    G = K // GROUP
    codes = torch.randint(0, 16, (N, K), generator=gen, device=device, dtype=torch.int32)
    scales = (0.005 + 0.015 * torch.rand(G, N, generator=gen, device=device)).to(torch.float16)
    zeros = torch.randint(6, 10, (G, N), generator=gen, device=device, dtype=torch.int32)
    qw = pack_awq(codes.t().contiguous())
    qz = pack_awq(zeros)
    return Weights(qw, scales, qz, codes.to(torch.uint8) if keep_codes else None, zeros)


def w16_scales(w: Weights) -> tuple[torch.Tensor, torch.Tensor]:
    """WQLinear's fp16 (scales, scaled_zeros) [G, N] for the same weights: scaled_zeros = -(s * z),
    rounded to fp16 as WQLinear.from_linear stores it (qmodule.py:199-203)."""
    sz = (-(w.awq_scales.float() * w.zeros.float())).to(torch.float16)
    return w.awq_scales, sz


@dataclass
class LinearSpec:
    name: str
    N: int
    K: int
    pairs: torch.Tensor
    theta: torch.Tensor
    channel_scales: torch.Tensor
    w: Weights


def linear_spec(name: str, N: int, K: int, gen: torch.Generator, device="cpu", keep_codes=False) -> LinearSpec:
    pairs, theta, cs = rotation_params(K, gen, device)
    return LinearSpec(name, N, K, pairs, theta, cs, weights(N, K, gen, device, keep_codes))


def build_module(spec: LinearSpec, device="cuda"):
    """BF16RotateLinearWrapper(RotateLinearInt4(..., qlinear=MarlinW4A8Linear)) on `device`."""
    from .quantization import BF16RotateLinearWrapper, MarlinW4A8Linear, RotateLinearInt4

    rl = RotateLinearInt4(spec.K, spec.N, bias=False, dtype=torch.float16,
                          rotation_angles=spec.theta.to(device), rotation_pairs=spec.pairs.to(device),
                          channel_scales=spec.channel_scales.to(device))
    rl = rl.to(device)
    q = MarlinW4A8Linear(spec.K, spec.N, GROUP)
    q.load_from_awq(spec.w.awq_qweight.to(device), spec.w.awq_scales.to(device), spec.w.awq_qzeros.to(device))
    rl.qlinear = q
    rl.rotation.prepare()
    return BF16RotateLinearWrapper(rl)


def ragged_lengths(n_requests: int, gen: torch.Generator, lo: int = 1, hi: int = 512) -> list[int]:
    return [int(v) for v in torch.randint(lo, hi + 1, (n_requests,), generator=gen)]


def build_w16_module(spec: LinearSpec, device="cuda"):
    """RotateLinearInt4(..., qlinear=WQLinear) on `device`, the W4A16 form of the same layer (needs the codes)."""
    from .quantization import RotateLinearInt4
    from .quantization.qmodule import pack_intweight

    if spec.w.codes is None:
        raise ValueError("build_w16_module needs a spec made with keep_codes=True")
    rl = RotateLinearInt4(spec.K, spec.N, bias=False, dtype=torch.float16,
                          rotation_angles=spec.theta.to(device), rotation_pairs=spec.pairs.to(device),
                          channel_scales=spec.channel_scales.to(device))
    rl = rl.to(device)
    q = rl.qlinear
    G = spec.K // GROUP
    s, sz = w16_scales(spec.w)
    q.qweight.copy_(pack_intweight(spec.w.codes.to(torch.int32)).to(device))
    q.scales[:G].copy_(s.to(device))
    q.scaled_zeros[:G].copy_(sz.to(device))
    q.prepare()
    rl.rotation.prepare()
    return rl
