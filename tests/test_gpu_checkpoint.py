"""A ParoQuant checkpoint end to end on the GPU: torch.save'd state dict (with out-of-range channel scales)
-> load_paroquant_checkpoint (weights_only) -> the W4A16 layers as loaded (grouped and alone) ->
convert_model_to_marlin_w4a8 -> every W4A8 layer against the oracle computed from the checkpoint's own
tensors (paroquant_marlin_w4a8.py:426-529; rotation_linear.py:120-124)."""

import pytest
import torch

import alpamayo_amd  # noqa: F401
from alpamayo_amd import workloads
from alpamayo_amd.quantization import (
    BF16RotateLinearWrapper,
    MarlinW4A8Linear,
    SharedInputRotateLinears,
    convert_model_to_marlin_w4a8,
    load_paroquant_checkpoint,
)
from oracle import linear as olin
from oracle import packing as opack
from oracle import rotation as orot
from oracle import w4a16 as ow
from tests.ckpt_util import LINEARS, PREFIX, ToyAlpamayo, paroquant_state_dict
from tests.gpu_util import assert_bf16_close, rel_fro, to_np

pytestmark = pytest.mark.gpu


def _ckpt(tmp_path):
    sd = paroquant_state_dict()
    q0 = f"{PREFIX}.0.self_attn.q_proj.rotation.channel_scales"
    sd[q0][0, :2] = float("inf")
    sd[q0][0, 2] = 2000.0
    path = tmp_path / "paroquant.pt"
    torch.save(sd, path)
    return path


def _oracle_operands(rl):
    """Codes, AWQ scales / zeros, rotation and bias of a loaded RotateLinearInt4, from its buffers, by the
    oracle's own unpacking (oracle/packing.py)."""
    q, r = rl.qlinear, rl.rotation
    N, K = q.out_features, q.in_features
    awq = opack.wqlinear_to_awq(q.qweight.cpu().numpy(), q.scales.cpu().numpy(), q.scaled_zeros.cpu().numpy(), N, K,
                                128)
    codes = opack.unpack_wqlinear_qweight(q.qweight.cpu().numpy(), N, K)
    c, s = orot.cos_sin_table(r.theta.cpu().numpy())
    bias = q.bias.float().cpu().numpy() if q.bias is not None else None
    return awq, codes, r.pairs.cpu().numpy(), c, s, r.channel_scales.float().cpu().numpy().reshape(-1), bias


def test_checkpoint_to_w4a16_and_w4a8_parity(tmp_path):
    model, rep = load_paroquant_checkpoint(ToyAlpamayo(), str(_ckpt(tmp_path)), device="cuda")
    assert rep.sanitised == 1 and rep.missing == [] and rep.zero_scales == []
    layers = model.vlm.model.language_model.layers
    g = workloads.generator(4100)
    xs = {K: workloads.activations(5, K, g).cuda() for K in (256, 384)}

    # As loaded: WQLinear (W4A16) behind the bf16 wrappers.  The q/k/v group equals the separate calls.
    attn = layers[0].self_attn
    grp = SharedInputRotateLinears([attn.q_proj, attn.k_proj, attn.v_proj])
    assert grp.w4a16
    outs = grp(xs[256])
    for y, mod in zip(outs, (attn.q_proj, attn.k_proj, attn.v_proj)):
        ref = mod(xs[256])
        assert y.dtype == torch.bfloat16
        assert rel_fro(to_np(y), to_np(ref)) < 1e-2
    # ... and the q projection (with bias and clipped scales) against the W4A16 oracle
    awq, codes, pairs, c, s, sc, bias = _oracle_operands(attn.q_proj.rotate_linear)
    wq = attn.q_proj.rotate_linear.qlinear
    ref16, _ = ow.rotate_linear_w16(to_np(xs[256]), pairs, c, s, sc, codes, wq.scales[:2].cpu().numpy(),
                                    wq.scaled_zeros[:2].cpu().numpy(), bias, input_fp16=True)
    assert rel_fro(to_np(attn.q_proj(xs[256])), ref16) < 1e-2
    assert sc[0] == 511.75 and sc[2] == 511.75            # the clipped channel scales are what runs

    # The oracle's operands of every layer, read from the loaded buffers before the WQLinear goes away.
    operands = {(li, name): _oracle_operands(getattr(getattr(layer, block), name).rotate_linear)
                for li, layer in enumerate(layers) for block, names in LINEARS.items() for name in names}
    # Converted to W4A8: every linear against the oracle.
    assert convert_model_to_marlin_w4a8(model) == 14
    for li, layer in enumerate(layers):
        for block, names in LINEARS.items():
            for name, (N, K) in names.items():
                mod = getattr(getattr(layer, block), name)
                assert isinstance(mod, BF16RotateLinearWrapper)
                assert isinstance(mod.rotate_linear.qlinear, MarlinW4A8Linear)
                print(f"checkpoint layer {li} {name}", flush=True)
                y = mod(xs[K])
                awq, codes, pairs, c, s, sc, bias = operands[(li, name)]
                ref, _, _ = olin.w4a8_rotate_linear(to_np(xs[K]), pairs, c, s, sc, codes, awq[1], awq[4], bias)
                assert_bf16_close(to_np(y), ref)
