"""ParoQuant checkpoint ingestion on the CPU (load_paroquant_model's checkpoint half,
paroquant_marlin_w4a8.py:462-510): a torch.save'd state dict read with weights_only, key diagnostics, the
all-zero-scales detector, the channel-scale clip and the bf16 wrapping."""

import logging
import math

import torch

import alpamayo_amd  # noqa: F401
from alpamayo_amd.quantization import BF16RotateLinearWrapper, RotateLinearInt4, load_paroquant_checkpoint
from alpamayo_amd.quantization.paroquant_marlin_w4a8 import _FP16_SAFE_SCALE
from tests.ckpt_util import PREFIX, ToyAlpamayo, paroquant_state_dict


def _damaged_checkpoint(tmp_path):
    sd = paroquant_state_dict()
    q0 = f"{PREFIX}.0.self_attn.q_proj.rotation.channel_scales"
    sd[q0][0, :3] = float("inf")
    sd[q0][0, 3:5] = 1000.0
    sd[q0][0, 5] = -float("inf")
    sd[f"{PREFIX}.1.self_attn.k_proj.rotation.channel_scales"][0, 7] = float("nan")
    del sd[f"{PREFIX}.1.self_attn.v_proj.qlinear.scales"]         # a quantized layer whose scales never load
    sd["extra.weight"] = torch.zeros(3)
    path = tmp_path / "paroquant.pt"
    torch.save(sd, path)
    return path, sd


def test_load_checkpoint_reports_and_sanitises(tmp_path, caplog):
    path, sd = _damaged_checkpoint(tmp_path)
    model = ToyAlpamayo()
    with caplog.at_level(logging.INFO, logger="alpamayo_amd.quantization.paroquant_marlin_w4a8"):
        model, rep = load_paroquant_checkpoint(model, str(path), device="cpu")
    v1 = f"{PREFIX}.1.self_attn.v_proj.qlinear.scales"
    assert rep.unexpected == ["extra.weight"]
    assert rep.missing == [v1] and rep.quant_missing == [v1]
    assert rep.zero_scales == [v1]
    assert rep.sanitised == 2
    assert any("all zero" in r.message for r in caplog.records if r.levelno == logging.ERROR)
    layers = model.vlm.model.language_model.layers
    # every quantized linear is wrapped for bf16 activations; lm_head (outside the layers) is untouched
    for layer in layers:
        for block in (layer.self_attn, layer.mlp):
            for _, child in block.named_children():
                assert isinstance(child, BF16RotateLinearWrapper)
                assert isinstance(child.rotate_linear, RotateLinearInt4)
    assert isinstance(model.vlm.lm_head, torch.nn.Linear)
    cs = layers[0].self_attn.q_proj.rotate_linear.rotation.channel_scales.float().reshape(-1)
    assert torch.all(cs[:3] == _FP16_SAFE_SCALE) and torch.all(cs[3:5] == _FP16_SAFE_SCALE)
    assert cs[5] == -_FP16_SAFE_SCALE
    orig = sd[f"{PREFIX}.0.self_attn.q_proj.rotation.channel_scales"].float().reshape(-1)
    assert torch.equal(cs[6:], orig[6:])
    k1 = layers[1].self_attn.k_proj.rotate_linear.rotation.channel_scales.float().reshape(-1)
    assert math.isnan(float(k1[7]))                                   # the clip cannot repair a NaN
    assert torch.equal(layers[0].input_layernorm.weight.detach(), sd[f"{PREFIX}.0.input_layernorm.weight"])
    assert not model.training


def test_load_checkpoint_from_dict_clean():
    model, rep = load_paroquant_checkpoint(ToyAlpamayo(), paroquant_state_dict(), device="cpu", wrap_bf16=False)
    assert rep.missing == [] and rep.unexpected == [] and rep.zero_scales == [] and rep.sanitised == 0
    q = model.vlm.model.language_model.layers[0].self_attn.q_proj
    assert isinstance(q, RotateLinearInt4) and q.qlinear.bias is not None
