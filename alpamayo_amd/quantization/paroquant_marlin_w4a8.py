"""ParoQuant W4A8 linear: converters and the quantized Linear module.

Mirrors src/alpamayo_r1/utils/quantization/paroquant_marlin_w4a8.py with the
same public names and signatures:

  BF16RotateLinearWrapper           (47-71)
  unpack_wqlinear_qweight           (95-142)
  _AWQ_ORDER, pack_awq_int32        (149-164)
  AWQBuffers, wqlinear_to_awq       (167-209)
  dequant_wqlinear, dequant_awq     (216-235)
  MarlinW4A8Linear                  (242-333): __init__(in, out, group_size),
                                    load_from_awq(qweight, scales, qzeros, bias), forward(x)
  convert_wqlinear_layer            (340-353)
  _wrap_rotate_linears, replace_linears_with_rotate_linear, _sanitise_channel_scales (356-423)
  convert_model_to_marlin_w4a8      (513-529)
  load_paroquant_checkpoint         (the checkpoint part of load_paroquant_model, 462-510)

Added here, with no counterpart in the reference: ``SharedInputRotateLinears``,
which runs linears that read one activation (q/k/v, gate/up) as one group
through ``paroquant::w4a8_linear_group``.

What changes underneath: ``load_from_awq`` repacks into this project's
kernel layout with ``paroquant::w4a8_prepack`` instead of vLLM's Marlin
repack, and ``forward`` runs ``paroquant::quant_i8`` + ``paroquant::w4a8_gemm``
(HIP kernels for gfx950) instead of ``apply_awq_marlin_linear``.  When a
``RotateLinearInt4`` owns a ``MarlinW4A8Linear``, rotation, quantization and
GEMM run as ``paroquant::w4a8_linear`` (two kernel launches).

Buffers of ``MarlinW4A8Linear`` (all registered, so graph capture sees fixed
addresses, as in the reference 262-271):
  qweight    uint8 [N/16, K/128, 64, 16]   packed int4 codes
  scales     int32 [N/16, K/128, 16]       fp16 group scale | zero point << 16
  qzeros     empty (zero points live in ``scales``)
  workspace  uint8                          scratch of paroquant::w4a8_linear for M <= 16
                                            (int8 codes and scales between its two kernels)
  g_idx, g_idx_sort_indices   empty int32 (no act-order), kept for API parity
  input_global_scale          float32 [1] = 1 (the fp16 scales are used as is)
"""

from __future__ import annotations

import logging
from typing import NamedTuple

import torch
import torch.nn as nn

from .. import ops as _ops
from .qmodule import WQLinear, unpack_intweight
from .rotation_linear import RotateLinearInt4, Rotation

logger = logging.getLogger(__name__)

_WORKSPACE_MAX_M = 16


# ---------------------------------------------------------------------------
# bf16 wrapper
# ---------------------------------------------------------------------------

class BF16RotateLinearWrapper(nn.Module):
    """Lets a RotateLinearInt4 take bfloat16 activations.

    The reference casts bf16 -> fp16, runs the fp16 rotation and GEMM and
    casts the result back.  With a MarlinW4A8Linear inside, this runs the
    fused kernels directly on the bf16 tensor: the kernel rounds the input to
    fp16 (the same cast), keeps the fp16-rounded rotation, and writes bf16.
    """

    def __init__(self, rotate_linear: nn.Module):
        super().__init__()
        self.rotate_linear = rotate_linear

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        rl = self.rotate_linear
        if isinstance(rl, RotateLinearInt4) and isinstance(rl.qlinear, MarlinW4A8Linear):
            return rl.qlinear.forward_rotated(x, rl.rotation, input_fp16=True, out_dtype=x.dtype)
        input_dtype = x.dtype
        with torch.amp.autocast("cuda", enabled=False):
            out = rl(x.to(torch.float16))
        return out.to(input_dtype)

    def __getattr__(self, name: str):
        try:
            return super().__getattr__(name)
        except AttributeError:
            return getattr(self.rotate_linear, name)


class SharedInputRotateLinears(nn.Module):
    """Linears that read the same activation -- q/k/v, or gate/up -- run as one group.

    Each member keeps its own rotation and weights; forward(x) returns the
    members' outputs, equal to calling each member on x.  The group runs
    paroquant::w4a8_linear_group: one rotation (+ quant) launch for all
    members and one GEMM launch over their concatenated output columns,
    where separate calls take two launches per linear.  Members are
    BF16RotateLinearWrapper or RotateLinearInt4 modules holding a
    MarlinW4A8Linear, all of one kind, with one in_features and one number
    of rotation layers.  The reference keeps these linears separate once
    ParoQuant is loaded (paroquant_marlin_w4a8.py:455-460); its unquantised
    counterparts are QKVLinear / MergedColumnLinear (patches.py:144-263).
    """

    def __init__(self, members):
        super().__init__()
        members = list(members)
        if not 1 <= len(members) <= _ops._lib.MAX_GROUP:
            raise ValueError(f"a group holds 1..{_ops._lib.MAX_GROUP} linears, got {len(members)}")
        kinds = {type(m) for m in members}
        if len(kinds) != 1 or not kinds <= {BF16RotateLinearWrapper, RotateLinearInt4}:
            raise TypeError("members must all be BF16RotateLinearWrapper or all RotateLinearInt4")
        rls = [m.rotate_linear if isinstance(m, BF16RotateLinearWrapper) else m for m in members]
        for rl in rls:
            if not isinstance(rl.qlinear, MarlinW4A8Linear):
                raise TypeError("every member must hold a MarlinW4A8Linear (convert_model_to_marlin_w4a8)")
        if len({rl.qlinear.in_features for rl in rls}) != 1 or len({rl.rotation.krot for rl in rls}) != 1:
            raise ValueError("members must share in_features and the number of rotation layers")
        self.members = nn.ModuleList(members)
        self.bf16_inputs = isinstance(members[0], BF16RotateLinearWrapper)
        self.register_buffer("workspace", torch.empty(0, dtype=torch.uint8), persistent=False)

    def _rotate_linears(self):
        return [m.rotate_linear if self.bf16_inputs else m for m in self.members]

    def _args(self, x):
        rls = self._rotate_linears()
        for rl in rls:
            rl.qlinear._check_loaded()
            if not rl.rotation.prepared:
                rl.rotation.prepare()
        k = x.size(-1)
        need = _ops.linear_group_workspace_bytes(x.numel() // k, k, len(rls))
        if self.workspace.numel() < need or self.workspace.device != x.device:
            self.workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
        return ([rl.rotation.rot_idx for rl in rls], [rl.rotation.rot_cs for rl in rls],
                [rl.rotation.scales_f32 for rl in rls], rls[0].rotation.krot, [rl.qlinear.qweight for rl in rls],
                [rl.qlinear.scales for rl in rls], [rl.qlinear.bias for rl in rls], self.workspace,
                self.bf16_inputs, True, x.dtype)

    def forward(self, x: torch.Tensor, norm_weight: torch.Tensor | None = None, eps: float = 1e-6,
                residual: torch.Tensor | None = None, return_normed: bool = False, return_sum: bool = False):
        """The members' outputs on x; with ``norm_weight``, on the decoder layer's RMSNorm of
        x (+ residual): h = weight * (s * rsqrt(mean(s^2) + eps)) with s = x + residual, in x's dtype
        (Qwen3VLTextRMSNorm.forward, modeling_qwen3_vl.py:354-359); with only ``residual``, on
        s = x + residual (a decoder layer's residual add).  The norm runs inside the group's rotation
        launch; the add does where the group runs the split rotation (decode sizes), and as a
        separate torch add otherwise, which measured faster there.  ``return_normed`` /
        ``return_sum`` append h / s to the outputs."""
        args = self._args(x)
        if norm_weight is not None:
            outs = torch.ops.paroquant.w4a8_linear_group_fused(x, residual, norm_weight.to(x.dtype), float(eps),
                                                               _ops._lib.PQ_PRO_RMSNORM, *args, return_normed,
                                                               return_sum)
        elif residual is not None:
            if return_normed:
                raise ValueError("return_normed needs norm_weight (the add alone returns its sum: return_sum)")
            if _ops.split_path(x.numel() // x.size(-1), x.size(-1)):
                outs = torch.ops.paroquant.w4a8_linear_group_fused(x, residual, None, 0.0, _ops._lib.PQ_PRO_ADD,
                                                                   *args, False, return_sum)
            else:   # the row kernel: a separate add is cheaper (same result bit for bit)
                s = x + residual
                outs = list(torch.ops.paroquant.w4a8_linear_group(s, *args)) + ([s] if return_sum else [])
        else:
            if return_normed or return_sum:
                raise ValueError("return_normed / return_sum need norm_weight or residual")
            outs = torch.ops.paroquant.w4a8_linear_group(x, *args)
        return tuple(outs)

    def forward_swiglu(self, gate: torch.Tensor, up: torch.Tensor, return_act: bool = False):
        """The members' outputs on act = silu(gate) * up in the inputs' dtype (a gated MLP's down_proj
        input, patches.py:541-548: silu in float32, rounded, times up, rounded), formed inside the
        group's rotation launch where the group runs the split rotation (decode sizes), by torch's
        silu and mul otherwise (measured faster there).  ``return_act`` appends act."""
        args = self._args(gate)
        if _ops.split_path(gate.numel() // gate.size(-1), gate.size(-1)):
            outs = torch.ops.paroquant.w4a8_linear_group_fused(gate, up, None, 0.0, _ops._lib.PQ_PRO_SWIGLU, *args,
                                                               return_act, False)
        else:   # the row kernel: separate elementwise kernels are cheaper (same rows, up to silu's last bit)
            act = torch.nn.functional.silu(gate) * up
            outs = list(torch.ops.paroquant.w4a8_linear_group(act, *args)) + ([act] if return_act else [])
        return tuple(outs)


def _get_alpamayo_layers(model, target="vlm"):
    if target == "expert":
        return model.expert.layers
    return model.vlm.model.language_model.layers


def _iter_linears(module, prefix=""):
    for name, child in module.named_children():
        full = f"{prefix}.{name}" if prefix else name
        if isinstance(child, nn.Linear):
            yield full, module, name, child
        yield from _iter_linears(child, full)


# ---------------------------------------------------------------------------
# weight formats
# ---------------------------------------------------------------------------

def unpack_wqlinear_qweight(qweight: torch.Tensor, out_features: int, in_features: int, interleave: int = 4,
                            kstride: int = 64) -> torch.Tensor:
    """WQLinear int16 [N/4, K] -> int4 codes [N, K] int32 in [0, 15]."""
    return unpack_intweight(qweight, out_features, in_features, interleave, kstride)


_AWQ_ORDER = [0, 2, 4, 6, 1, 3, 5, 7]


def pack_awq_int32(values: torch.Tensor) -> torch.Tensor:
    """[rows, cols] int4 -> [rows, cols/8] int32; nibble i holds column 8c + _AWQ_ORDER[i]."""
    rows, cols = values.shape
    assert cols % 8 == 0, f"cols={cols} must be divisible by 8"
    v = values.to(torch.int32).reshape(rows, cols // 8, 8)
    packed = torch.zeros(rows, cols // 8, dtype=torch.int32, device=values.device)
    for i, src in enumerate(_AWQ_ORDER):
        packed |= (v[:, :, src] & 0xF) << (4 * i)
    return packed


def unpack_awq_int32(packed: torch.Tensor, cols: int) -> torch.Tensor:
    """Inverse of pack_awq_int32 -> [rows, cols] int32."""
    rows = packed.shape[0]
    out = torch.empty(rows, cols // 8, 8, dtype=torch.int32, device=packed.device)
    for i, dst in enumerate(_AWQ_ORDER):
        out[:, :, dst] = (packed >> (4 * i)) & 0xF
    return out.reshape(rows, cols)


class AWQBuffers(NamedTuple):
    qweight: torch.Tensor      # (K, N//8) int32
    scales: torch.Tensor       # (num_groups, N) float16
    qzeros: torch.Tensor       # (num_groups, N//8) int32
    int4_values: torch.Tensor  # (N, K) int32
    zeros: torch.Tensor        # (num_groups, N) int32


def wqlinear_to_awq(qweight_i16, scales, scaled_zeros, out_features, in_features, group_size) -> AWQBuffers:
    """WQLinear buffers -> AWQ buffers; zeros recovered as round(-scaled_zeros / scales) in [0, 15]."""
    N, K = out_features, in_features
    G = K // group_size
    int4 = unpack_wqlinear_qweight(qweight_i16, N, K)
    awq_qweight = pack_awq_int32(int4.t().contiguous())
    awq_scales = scales[:G, :N].contiguous().to(torch.float16)
    safe = awq_scales.float().clone()
    safe[safe.abs() < 1e-10] = 1.0
    zeros = (-scaled_zeros[:G, :N].float() / safe).round().clamp(0, 15).to(torch.int32)
    return AWQBuffers(awq_qweight, awq_scales, pack_awq_int32(zeros), int4, zeros)


def dequant_wqlinear(int4_NK, scales, scaled_zeros, group_size):
    """w = q * s + sz."""
    N, K = int4_NK.shape
    G = K // group_size
    sc = scales[:G, :N].float().repeat_interleave(group_size, dim=0).t()
    sz = scaled_zeros[:G, :N].float().repeat_interleave(group_size, dim=0).t()
    return int4_NK.float() * sc + sz


def dequant_awq(int4_NK, zeros, scales, group_size):
    """w = (q - z) * s."""
    N, K = int4_NK.shape
    G = K // group_size
    sc = scales[:G, :N].float().repeat_interleave(group_size, dim=0).t()
    zp = zeros[:G, :N].float().repeat_interleave(group_size, dim=0).t()
    return (int4_NK.float() - zp) * sc


# ---------------------------------------------------------------------------
# the quantized Linear
# ---------------------------------------------------------------------------

class MarlinW4A8Linear(nn.Module):
    """int4 weights (group 128, zero points) x per-token int8 activations."""

    def __init__(self, in_features: int, out_features: int, group_size: int = 128):
        super().__init__()
        if group_size != 128:
            raise NotImplementedError("only group_size=128 is supported")
        if in_features % 128 or out_features % 16:
            raise ValueError("in_features must be a multiple of 128 and out_features of 16")
        self.in_features = in_features
        self.out_features = out_features
        self.group_size = group_size
        self.register_buffer("qweight", torch.empty(0, dtype=torch.uint8))
        self.register_buffer("scales", torch.empty(0, dtype=torch.int32))
        self.register_buffer("qzeros", torch.empty(0, dtype=torch.int32))
        self.register_buffer("workspace", torch.empty(0, dtype=torch.uint8))
        self.register_buffer("g_idx", torch.empty(0, dtype=torch.int32))
        self.register_buffer("g_idx_sort_indices", torch.empty(0, dtype=torch.int32))
        self.register_buffer("input_global_scale", torch.ones(1, dtype=torch.float32))
        # registered up front so load_from_awq can assign it (the reference's
        # register_buffer after `self.bias = None` raises KeyError for biased layers)
        self.register_buffer("bias", None)

    @torch.no_grad()
    def load_from_awq(self, awq_qweight, awq_scales, awq_qzeros, bias=None):
        """AWQ int32 buffers -> kernel layout (on the inputs' device)."""
        dev = awq_qweight.device
        K, N = self.in_features, self.out_features
        if tuple(awq_qweight.shape) != (K, N // 8):
            raise ValueError(f"awq_qweight must be [{K}, {N // 8}], got {tuple(awq_qweight.shape)}")
        wpack, wmeta = torch.ops.paroquant.w4a8_prepack(
            awq_qweight.to(torch.int32).contiguous(), awq_scales.to(torch.float16).contiguous(),
            awq_qzeros.to(torch.int32).contiguous())
        self.qweight = wpack
        self.scales = wmeta
        self.qzeros = torch.empty(0, dtype=torch.int32, device=dev)
        self.g_idx = torch.empty(0, dtype=torch.int32, device=dev)
        self.g_idx_sort_indices = torch.empty(0, dtype=torch.int32, device=dev)
        self.input_global_scale = torch.ones(1, dtype=torch.float32, device=dev)
        ws = max(max(_ops.workspace_bytes(m, N, K), _ops.linear_workspace_bytes(m, N, K, 16))
                 for m in range(1, _WORKSPACE_MAX_M + 1))
        self.workspace = torch.zeros(max(ws, 1), dtype=torch.uint8, device=dev)
        self.bias = bias.to(dev).contiguous() if bias is not None else None

    def _check_loaded(self):
        if self.qweight.numel() == 0:
            raise RuntimeError("MarlinW4A8Linear: call load_from_awq() before forward()")

    @torch.no_grad()
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """x: already-rotated activations [..., K]; returns x.dtype [..., N]."""
        self._check_loaded()
        shape = x.shape
        xq, xs = torch.ops.paroquant.quant_i8(x.reshape(-1, shape[-1]))
        y = torch.ops.paroquant.w4a8_gemm(xq, xs, self.qweight, self.scales, self.bias, self.workspace, x.dtype)
        return y.view(*shape[:-1], self.out_features)

    @torch.no_grad()
    def forward_rotated(self, x: torch.Tensor, rotation: Rotation, input_fp16: bool, out_dtype: torch.dtype,
                        materialize_fp16: bool = True) -> torch.Tensor:
        """Rotation + int8 quant + GEMM on un-rotated activations x [..., K]."""
        self._check_loaded()
        if not rotation.prepared:
            rotation.prepare()
        return torch.ops.paroquant.w4a8_linear(
            x, rotation.rot_idx, rotation.rot_cs, rotation.scales_f32, rotation.krot, self.qweight, self.scales,
            self.bias, self.workspace, input_fp16, materialize_fp16, out_dtype)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, group_size={self.group_size}"


# ---------------------------------------------------------------------------
# converters
# ---------------------------------------------------------------------------

def convert_wqlinear_layer(qweight_i16, scales, scaled_zeros, out_features, in_features, group_size, bias=None,
                           device="cuda"):
    """WQLinear buffers -> (MarlinW4A8Linear on `device`, AWQBuffers)."""
    awq = wqlinear_to_awq(qweight_i16, scales, scaled_zeros, out_features, in_features, group_size)
    mod = MarlinW4A8Linear(in_features, out_features, group_size)
    mod.load_from_awq(awq.qweight.to(device), awq.scales.to(device), awq.qzeros.to(device),
                      bias=bias.to(device) if bias is not None else None)
    return mod, awq


def _wrap_rotate_linears(model, target="vlm"):
    for layer in _get_alpamayo_layers(model, target):
        for _, child in layer.named_children():
            for sub_name, sub_child in child.named_children():
                if isinstance(sub_child, RotateLinearInt4):
                    setattr(child, sub_name, BF16RotateLinearWrapper(sub_child))


def replace_linears_with_rotate_linear(model, target="vlm", init_only: bool = True,
                                       ignore_suffix: tuple[str, ...] = ("lm_head",)):
    """Replace every nn.Linear of the target layers by an empty RotateLinearInt4 shell."""
    for layer in _get_alpamayo_layers(model, target):
        for _, parent, child_name, linear in list(_iter_linears(layer)):
            if child_name in ignore_suffix:
                continue
            setattr(parent, child_name, RotateLinearInt4(
                in_feat=linear.in_features, out_feat=linear.out_features, bias=linear.bias is not None,
                dtype=torch.float16))


def _sanitise_channel_scales(model):
    """Clamp inf/NaN/|s| > 65504/128 channel scales (fp16 overflow guard)."""
    safe_max = 65504.0 / 128.0
    n_fixed = 0
    for name, mod in model.named_modules():
        if not isinstance(mod, RotateLinearInt4):
            continue
        cs = mod.rotation.channel_scales
        bad = torch.isinf(cs) | torch.isnan(cs) | (cs.abs() > safe_max)
        n_bad = int(bad.sum().item())
        if n_bad:
            with torch.no_grad():
                cs.clamp_(-safe_max, safe_max)   # like the reference, NaN entries stay NaN
            n_fixed += 1
            logger.warning("  Clamped %d/%d channel_scales in %s (had INF/NaN/overflow values)", n_bad,
                           cs.numel(), name)
    if n_fixed:
        logger.warning("Sanitised channel_scales in %d RotateLinearInt4 modules", n_fixed)
    return n_fixed


def load_paroquant_checkpoint(model, paro_checkpoint, *, target="vlm", device="cuda", wrap_bf16=True):
    """Put a ParoQuant state dict into an already-built model (load_paroquant_model 462-510)."""
    replace_linears_with_rotate_linear(model, target=target, init_only=True)
    sd = torch.load(paro_checkpoint, map_location="cpu", weights_only=True) if isinstance(paro_checkpoint, str) \
        else paro_checkpoint
    missing, unexpected = model.load_state_dict(sd, strict=False)
    quant_missing = [k for k in missing if any(s in k for s in ("qlinear", "rotation", "qweight", "scales",
                                                               "scaled_zeros"))]
    if quant_missing:
        logger.warning("CRITICAL quant missing: %s", quant_missing[:10])
    if unexpected:
        logger.warning("Unexpected keys (%d): %s", len(unexpected), unexpected[:20])
    _sanitise_channel_scales(model)
    if wrap_bf16:
        _wrap_rotate_linears(model, target=target)
    model.to(device)
    model.eval()
    return model, missing, unexpected


def convert_model_to_marlin_w4a8(model):
    """Replace the WQLinear of every RotateLinearInt4 by a MarlinW4A8Linear; returns the count."""
    n = 0
    for _, mod in model.named_modules():
        if not isinstance(mod, RotateLinearInt4):
            continue
        wq = mod.qlinear
        if not isinstance(wq, WQLinear):
            continue
        marlin, _ = convert_wqlinear_layer(wq.qweight.data, wq.scales.data, wq.scaled_zeros.data, wq.out_features,
                                           wq.in_features, wq.group_size, bias=wq.bias, device=wq.qweight.device)
        mod.qlinear = marlin
        mod.rotation.prepare()
        n += 1
    logger.info("Converted %d WQLinear -> MarlinW4A8Linear", n)
    return n
