"""A toy model with AlpamayoR1's module paths around two Qwen3-style decoder layers, and a ParoQuant state
dict for it built the offline way (RotateLinearInt4.from_linear, rotation_linear.py:68-118), for the
checkpoint-ingestion tests (load_paroquant_model, paroquant_marlin_w4a8.py:426-510).  Test infrastructure."""

from __future__ import annotations

import torch
import torch.nn as nn

from alpamayo_amd import workloads
from alpamayo_amd.quantization import RotateLinearInt4

H, KV, INTER = 256, 128, 384
LINEARS = {"self_attn": {"q_proj": (H, H), "k_proj": (KV, H), "v_proj": (KV, H), "o_proj": (H, H)},
           "mlp": {"gate_proj": (INTER, H), "up_proj": (INTER, H), "down_proj": (H, INTER)}}
PREFIX = "vlm.model.language_model.layers"


class _Block(nn.Module):
    def __init__(self, names):
        super().__init__()
        for n, (out_f, in_f) in names.items():
            setattr(self, n, nn.Linear(in_f, out_f, bias=(n == "q_proj")))


class _Layer(nn.Module):
    def __init__(self):
        super().__init__()
        self.self_attn = _Block(LINEARS["self_attn"])
        self.mlp = _Block(LINEARS["mlp"])
        self.input_layernorm = nn.Module()
        self.input_layernorm.weight = nn.Parameter(torch.ones(H))


class ToyAlpamayo(nn.Module):
    """model.vlm.model.language_model.layers[i].{self_attn,mlp}.<linear>, plus an lm_head outside the layers."""

    def __init__(self, n_layers=2):
        super().__init__()
        self.vlm = nn.Module()
        self.vlm.model = nn.Module()
        self.vlm.model.language_model = nn.Module()
        self.vlm.model.language_model.layers = nn.ModuleList([_Layer() for _ in range(n_layers)])
        self.vlm.lm_head = nn.Linear(H, 64, bias=False)


def paroquant_state_dict(n_layers=2, seed=77):
    """Quantized layers made offline from seeded fp weights and rotations; also the layer norms and lm_head."""
    g = workloads.generator(seed)
    sd = {}
    for li in range(n_layers):
        for block, names in LINEARS.items():
            for n, (out_f, in_f) in names.items():
                lin = nn.Linear(in_f, out_f, bias=(n == "q_proj"))
                with torch.no_grad():
                    lin.weight.copy_(torch.randn(out_f, in_f, generator=g) * 0.05)
                    if lin.bias is not None:
                        lin.bias.copy_(torch.randn(out_f, generator=g) * 0.1)
                pairs, theta, cs = workloads.rotation_params(in_f, g)
                rl = RotateLinearInt4.from_linear(lin, rotation_angles=theta, rotation_pairs=pairs,
                                                  channel_scales=cs, rotate_weight=True, init_only=False)
                for k, v in rl.state_dict().items():
                    sd[f"{PREFIX}.{li}.{block}.{n}.{k}"] = v.clone()
        sd[f"{PREFIX}.{li}.input_layernorm.weight"] = 0.8 + 0.4 * torch.rand(H, generator=g)
    sd["vlm.lm_head.weight"] = torch.randn(64, H, generator=g)
    return sd
