"""The integration guide's drop-in snippet for load_paroquant_model (paroquant_marlin_w4a8.py:426-510), executed as
the document writes it, on a toy model with AlpamayoR1's module paths (tests/ckpt_util.py): the checkpoint
load on the CPU, the whole block (load, then convert_model_to_marlin_w4a8) on the GPU."""

import os
import re

import pytest
import torch

import alpamayo_amd  # noqa: F401
from alpamayo_amd.quantization import BF16RotateLinearWrapper, MarlinW4A8Linear
from tests.ckpt_util import ToyAlpamayo, paroquant_state_dict

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GUIDE = os.path.join(ROOT, "INTEGRATION.md")


def _snippet():
    text = open(GUIDE).read()
    blocks = re.findall(r"```python\n(.*?)```", text, flags=re.S)
    found = [b for b in blocks if "load_paroquant_checkpoint(" in b and "convert_model_to_marlin_w4a8(" in b]
    assert len(found) == 1, "the guide holds one load -> convert block"
    return found[0]


def _run(code, device):
    ns = {"model": ToyAlpamayo(), "paro_checkpoint": paroquant_state_dict(), "device": device}
    exec(compile(code, GUIDE, "exec"), ns)   # noqa: S102 -- the guide's own code
    return ns


def test_snippet_load_lines_on_cpu():
    code = _snippet()
    lines = code.splitlines()
    cut = next(i for i, l in enumerate(lines) if l.startswith("convert_model_to_marlin_w4a8("))
    ns = _run("\n".join(lines[:cut]) + "\n", "cpu")
    rep = ns["report"]
    assert rep.missing == [] and rep.unexpected == [] and rep.zero_scales == [] and rep.sanitised == 0
    layer = ns["model"].vlm.model.language_model.layers[0]
    assert isinstance(layer.self_attn.q_proj, BF16RotateLinearWrapper)


@pytest.mark.gpu
def test_snippet_whole_block_on_gpu():
    ns = _run(_snippet(), "cuda")
    model = ns["model"]
    conv = [m for m in model.modules() if isinstance(m, MarlinW4A8Linear)]
    assert len(conv) == 14                                   # 2 layers x 7 linears
    q = model.vlm.model.language_model.layers[0].self_attn.q_proj
    x = torch.randn(3, q.rotate_linear.in_features, device="cuda").to(torch.bfloat16)
    y = q(x)
    assert y.shape == (3, q.rotate_linear.out_features) and y.dtype == torch.bfloat16
    assert torch.isfinite(y.float()).all()
