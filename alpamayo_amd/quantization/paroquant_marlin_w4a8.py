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
  workspace  empty uint8 (the ops take their scratch from torch's allocator), kept for API parity
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

# The longest rows the fused linear kernels take; longer ones run rotate -> quant -> GEMM as three ops.
_FUSED_MAX_K = 16384

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


def _rmsnorm_like_module(s: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """Qwen3VLTextRMSNorm.forward (modeling_qwen3_vl.py:354-359) with torch ops: float32 mean square and
    rsqrt, the normalized row rounded to s's dtype, then times the weight in that dtype."""
    sf = s.float()
    normed = (sf * torch.rsqrt(sf.pow(2).mean(-1, keepdim=True) + eps)).to(s.dtype)
    return weight.to(s.dtype) * normed


class SharedInputRotateLinears(nn.Module):
    """Linears that read the same activation -- q/k/v, or gate/up -- run as one group.

    Each member keeps its own rotation and weights; forward(x) returns the
    members' outputs, equal to calling each member on x.  Members are
    BF16RotateLinearWrapper or RotateLinearInt4 modules (all of one kind)
    with one in_features and one number of rotation layers, holding
    MarlinW4A8Linear weights (W4A8: paroquant::w4a8_linear_group, one
    rotation + quant launch for all members and one GEMM launch over their
    concatenated output columns, where separate calls take two launches per
    linear) or all WQLinear weights (W4A16: paroquant::w4a16_linear_group,
    one rotation launch and, up to 16 tokens, one GEMM launch).  The reference
    keeps these linears separate once ParoQuant is loaded
    (paroquant_marlin_w4a8.py:455-460); its unquantised counterparts are
    QKVLinear / MergedColumnLinear (patches.py:144-263).
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
        weight_kinds = {type(rl.qlinear) for rl in rls}
        if weight_kinds not in ({MarlinW4A8Linear}, {WQLinear}):
            raise TypeError("members must all hold MarlinW4A8Linear (convert_model_to_marlin_w4a8) or all WQLinear")
        if len({rl.qlinear.in_features for rl in rls}) != 1 or len({rl.rotation.krot for rl in rls}) != 1:
            raise ValueError("members must share in_features and the number of rotation layers")
        self.members = nn.ModuleList(members)
        self.bf16_inputs = isinstance(members[0], BF16RotateLinearWrapper)
        self.w4a16 = weight_kinds == {WQLinear}

    def _rotate_linears(self):
        return [m.rotate_linear if self.bf16_inputs else m for m in self.members]

    def _args(self, x):
        rls = self._rotate_linears()
        if not torch.compiler.is_compiling():
            # Host-side checks run eagerly only: under torch.compile the members must have been prepared
            # (prepare(), or one eager call).
            for rl in rls:
                if self.w4a16:
                    if not rl.qlinear.prepared:
                        rl.qlinear.prepare()
                else:
                    rl.qlinear._check_loaded()
                if not rl.rotation.prepared:
                    rl.rotation.prepare()
        rot = ([rl.rotation.rot_idx for rl in rls], [rl.rotation.rot_cs for rl in rls],
               [rl.rotation.scales_f32 for rl in rls], rls[0].rotation.krot)
        if self.w4a16:
            return rot + ([rl.qlinear.w16_pack for rl in rls], [rl.qlinear.w16_meta for rl in rls],
                          [rl.qlinear.bias for rl in rls], self.bf16_inputs, x.dtype)
        return rot + ([rl.qlinear.qweight for rl in rls], [rl.qlinear.scales for rl in rls],
                      [rl.qlinear.bias for rl in rls], self.bf16_inputs, True, x.dtype)

    def _plain(self, x):
        if self.w4a16:
            return list(torch.ops.paroquant.w4a16_linear_group(x, *self._args(x)))
        return list(torch.ops.paroquant.w4a8_linear_group(x, *self._args(x)))

    def forward(self, x: torch.Tensor, norm_weight: torch.Tensor | None = None, eps: float = 1e-6,
                residual: torch.Tensor | None = None, return_normed: bool = False, return_sum: bool = False):
        """The members' outputs on x; with ``norm_weight``, on the decoder layer's RMSNorm of
        x (+ residual): h = weight * (s * rsqrt(mean(s^2) + eps)) with s = x + residual, in x's dtype
        (Qwen3VLTextRMSNorm.forward, modeling_qwen3_vl.py:354-359); with only ``residual``, on
        s = x + residual (a decoder layer's residual add).  With W4A8 members the norm runs inside the
        group's rotation launch, and so does the add where the group runs the split rotation (decode
        sizes; a separate torch add measured faster otherwise); with W4A16 members both are torch ops.
        ``return_normed`` / ``return_sum`` append h / s to the outputs."""
        if return_normed and norm_weight is None:
            raise ValueError("return_normed needs norm_weight (the add alone returns its sum: return_sum)")
        if return_sum and residual is None:
            raise ValueError("return_sum needs a residual")
        k = x.size(-1)
        if self.w4a16:
            s = x + residual if residual is not None else x
            h = _rmsnorm_like_module(s, norm_weight, eps) if norm_weight is not None else s
            return tuple(self._plain(h) + ([h] if return_normed else []) + ([s] if return_sum else []))
        if norm_weight is not None:
            outs = torch.ops.paroquant.w4a8_linear_group_fused(x, residual, norm_weight.to(x.dtype), float(eps),
                                                               _ops._lib.PQ_PRO_RMSNORM, *self._args(x),
                                                               return_normed, return_sum)
        elif residual is not None:
            if _ops.split_path(x.numel() // k, k):
                outs = torch.ops.paroquant.w4a8_linear_group_fused(x, residual, None, 0.0, _ops._lib.PQ_PRO_ADD,
                                                                   *self._args(x), False, return_sum)
            else:   # the row kernel: a separate add is cheaper (same result bit for bit)
                s = x + residual
                outs = self._plain(s) + ([s] if return_sum else [])
        else:
            outs = self._plain(x)
        return tuple(outs)

    def forward_swiglu(self, gate: torch.Tensor, up: torch.Tensor, return_act: bool = False):
        """The members' outputs on act = silu(gate) * up in the inputs' dtype (a gated MLP's down_proj
        input, patches.py:541-548: silu in float32, rounded, times up, rounded), formed inside the
        group's rotation launch where W4A8 members run the split rotation (decode sizes), by torch's
        silu and mul otherwise (measured faster there).  ``return_act`` appends act."""
        k = gate.size(-1)
        if not self.w4a16 and _ops.split_path(gate.numel() // k, k):
            outs = torch.ops.paroquant.w4a8_linear_group_fused(gate, up, None, 0.0, _ops._lib.PQ_PRO_SWIGLU,
                                                               *self._args(gate), return_act, False)
        else:   # separate elementwise kernels (same rows, up to silu's last bit)
            act = torch.nn.functional.silu(gate) * up
            outs = self._plain(act) + ([act] if return_act else [])
        return tuple(outs)


def _get_alpamayo_layers(model, target="vlm"):
    """The decoder layers whose linears ParoQuant replaces: the language model's (target "vlm") or the action
    expert's ("expert"), at the module paths of AlpamayoR1 (paroquant_marlin_w4a8.py:74-80)."""
    root = model.expert if target == "expert" else model.vlm.model.language_model
    return root.layers


def _modules_with_parent(root: nn.Module, kind):
    """(parent, attribute name, module) for every submodule of `kind` below `root`, collected before any
    replacement so the caller may swap them in place."""
    found = []
    for parent in root.modules():
        for name, child in parent.named_children():
            if isinstance(child, kind):
                found.append((parent, name, child))
    return found


# ---------------------------------------------------------------------------
# weight formats
# ---------------------------------------------------------------------------

def unpack_wqlinear_qweight(qweight: torch.Tensor, out_features: int, in_features: int, interleave: int = 4,
                            kstride: int = 64) -> torch.Tensor:
    """WQLinear int16 [N/4, K] -> int4 codes [N, K] int32 in [0, 15]."""
    return unpack_intweight(qweight, out_features, in_features, interleave, kstride)


# AWQ's int32 word c of a row holds the 8 columns 8c .. 8c+7; nibble i (bits 4i .. 4i+3) holds column
# 8c + _AWQ_ORDER[i].  _AWQ_NIBBLE_OF is the inverse: the nibble that holds column 8c + j.
_AWQ_ORDER = [0, 2, 4, 6, 1, 3, 5, 7]
_AWQ_NIBBLE_OF = [_AWQ_ORDER.index(j) for j in range(8)]


def _nibble_shifts(device) -> torch.Tensor:
    return torch.arange(0, 32, 4, dtype=torch.int64, device=device)


def pack_awq_int32(values: torch.Tensor) -> torch.Tensor:
    """[rows, cols] int4 -> [rows, cols/8] int32 in AWQ's nibble order."""
    rows, cols = values.shape
    if cols % 8:
        raise ValueError(f"cols={cols} must be divisible by 8")
    nib = (values.to(torch.int64) & 0xF).reshape(rows, cols // 8, 8)[:, :, _AWQ_ORDER]
    word = (nib << _nibble_shifts(values.device)).sum(dim=-1)          # disjoint nibbles: sum == or
    return torch.where(word >= 2 ** 31, word - 2 ** 32, word).to(torch.int32)


def unpack_awq_int32(packed: torch.Tensor, cols: int) -> torch.Tensor:
    """Inverse of pack_awq_int32 -> [rows, cols] int32."""
    rows = packed.shape[0]
    nib = (packed.to(torch.int64).unsqueeze(-1) >> _nibble_shifts(packed.device)) & 0xF
    return nib[:, :, _AWQ_NIBBLE_OF].reshape(rows, cols).to(torch.int32)


class AWQBuffers(NamedTuple):
    qweight: torch.Tensor      # (K, N//8) int32
    scales: torch.Tensor       # (num_groups, N) float16
    qzeros: torch.Tensor       # (num_groups, N//8) int32
    int4_values: torch.Tensor  # (N, K) int32
    zeros: torch.Tensor        # (num_groups, N) int32


def wqlinear_to_awq(qweight_i16, scales, scaled_zeros, out_features, in_features, group_size) -> AWQBuffers:
    """WQLinear buffers -> AWQ buffers (paroquant_marlin_w4a8.py:179-209).

    WQLinear keeps the zero point only as scaled_zeros = -(s * z) in fp16 (qmodule.py:199-203); the integer
    zero point comes back as round(-scaled_zeros / s), clamped to the 4-bit range, with a zero scale (an
    unused group) read as 1.  Only the first K / group_size rows of WQLinear's padded scale buffers are used.
    """
    n_groups = in_features // group_size
    codes = unpack_wqlinear_qweight(qweight_i16, out_features, in_features)             # [N, K]
    s16 = scales[:n_groups, :out_features].to(torch.float16).contiguous()
    s32 = s16.float()
    denom = torch.where(s32.abs() < 1e-10, torch.ones_like(s32), s32)
    zeros = torch.clamp(torch.round(-scaled_zeros[:n_groups, :out_features].float() / denom), 0, 15)
    zeros = zeros.to(torch.int32)
    return AWQBuffers(qweight=pack_awq_int32(codes.t().contiguous()), scales=s16, qzeros=pack_awq_int32(zeros),
                      int4_values=codes, zeros=zeros)


def _per_group(t: torch.Tensor, n_out: int, n_groups: int) -> torch.Tensor:
    """[groups(+padding), N] -> float32 [N, groups, 1], to broadcast over a group's channels."""
    return t[:n_groups, :n_out].float().t().unsqueeze(-1)


def dequant_wqlinear(int4_NK, scales, scaled_zeros, group_size):
    """WQLinear's weights w = q * s + sz in float32, [N, K] (paroquant_marlin_w4a8.py:216-224)."""
    N, K = int4_NK.shape
    G = K // group_size
    q = int4_NK.float().reshape(N, G, group_size)
    return (q * _per_group(scales, N, G) + _per_group(scaled_zeros, N, G)).reshape(N, K)


def dequant_awq(int4_NK, zeros, scales, group_size):
    """AWQ's weights w = (q - z) * s in float32, [N, K] (paroquant_marlin_w4a8.py:227-235)."""
    N, K = int4_NK.shape
    G = K // group_size
    q = int4_NK.float().reshape(N, G, group_size)
    return ((q - _per_group(zeros, N, G)) * _per_group(scales, N, G)).reshape(N, K)


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
        self.workspace = torch.empty(0, dtype=torch.uint8, device=dev)
        self.bias = bias.to(dev).contiguous() if bias is not None else None

    def _check_loaded(self):
        if self.qweight.numel() == 0:
            raise RuntimeError("MarlinW4A8Linear: call load_from_awq() before forward()")

    @torch.no_grad()
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """x: already-rotated activations [..., K]; returns x.dtype [..., N]."""
        if not torch.compiler.is_compiling():
            self._check_loaded()
        shape = x.shape
        xq, xs = torch.ops.paroquant.quant_i8(x.reshape(-1, shape[-1]))
        y = torch.ops.paroquant.w4a8_gemm(xq, xs, self.qweight, self.scales, self.bias, x.dtype)
        return y.view(*shape[:-1], self.out_features)

    @torch.no_grad()
    def forward_rotated(self, x: torch.Tensor, rotation: Rotation, input_fp16: bool, out_dtype: torch.dtype,
                        materialize_fp16: bool = True) -> torch.Tensor:
        """Rotation + int8 quant + GEMM on un-rotated activations x [..., K].  Eagerly it checks that the
        weights are loaded and (re)prepares the rotation's operands when they are stale; under torch.compile
        it expects a prepared rotation (prepare(), or one eager call)."""
        if self.in_features > _FUSED_MAX_K:
            return self._forward_unfused(x, rotation, input_fp16, out_dtype, materialize_fp16)
        if not torch.compiler.is_compiling():
            self._check_loaded()
            if not rotation.prepared:
                rotation.prepare()
        return torch.ops.paroquant.w4a8_linear(
            x, rotation.rot_idx, rotation.rot_cs, rotation.scales_f32, rotation.krot, self.qweight, self.scales,
            self.bias, input_fp16, materialize_fp16, out_dtype)

    def _forward_unfused(self, x, rotation, input_fp16, out_dtype, materialize_fp16):
        """The same computation as paroquant::w4a8_linear in three ops, for rows longer than its kernels take
        (K > 16384): rotation::rotate in float32 (from x rounded to fp16 when input_fp16), the result rounded
        to fp16 when materialize_fp16, per-token int8 quantization, the GEMM."""
        if not torch.compiler.is_compiling():
            self._check_loaded()
        xin = x.to(torch.float16) if input_fp16 else x
        xr = torch.ops.rotation.rotate(xin.float(), rotation.pairs, rotation.theta.float(),
                                       rotation.channel_scales.float(), rotation.group_size)
        if materialize_fp16:
            xr = xr.to(torch.float16)
        xq, xs = torch.ops.paroquant.quant_i8(xr.reshape(-1, self.in_features))
        y = torch.ops.paroquant.w4a8_gemm(xq, xs, self.qweight, self.scales, self.bias, out_dtype)
        return y.view(*x.shape[:-1], self.out_features)

    def extra_repr(self) -> str:
        return f"in_features={self.in_features}, out_features={self.out_features}, group_size={self.group_size}"


# ---------------------------------------------------------------------------
# converters and checkpoint loading
# ---------------------------------------------------------------------------

def convert_wqlinear_layer(qweight_i16, scales, scaled_zeros, out_features, in_features, group_size, bias=None,
                           device="cuda"):
    """One WQLinear's buffers -> (a loaded MarlinW4A8Linear on `device`, the intermediate AWQBuffers)
    (paroquant_marlin_w4a8.py:340-353)."""
    awq = wqlinear_to_awq(qweight_i16, scales, scaled_zeros, out_features, in_features, group_size)
    layer = MarlinW4A8Linear(in_features, out_features, group_size)
    on_dev = [t.to(device) for t in (awq.qweight, awq.scales, awq.qzeros)]
    layer.load_from_awq(*on_dev, bias=None if bias is None else bias.to(device))
    return layer, awq


def _wrap_rotate_linears(model, target="vlm"):
    """Put every RotateLinearInt4 of the target layers behind a BF16RotateLinearWrapper (bf16 model,
    fp16 kernels; paroquant_marlin_w4a8.py:356-363)."""
    for layer in _get_alpamayo_layers(model, target):
        for parent, name, rl in _modules_with_parent(layer, RotateLinearInt4):
            if not isinstance(parent, BF16RotateLinearWrapper):
                setattr(parent, name, BF16RotateLinearWrapper(rl))


def replace_linears_with_rotate_linear(model, target="vlm", init_only: bool = True,
                                       ignore_suffix: tuple[str, ...] = ("lm_head",)):
    """Swap each nn.Linear of the target layers (except those named in ignore_suffix) for an empty fp16
    RotateLinearInt4 of the same shape, to be filled by load_state_dict (paroquant_marlin_w4a8.py:366-387)."""
    for layer in _get_alpamayo_layers(model, target):
        for parent, name, lin in _modules_with_parent(layer, nn.Linear):
            if name in ignore_suffix:
                continue
            shell = RotateLinearInt4(in_feat=lin.in_features, out_feat=lin.out_features, bias=lin.bias is not None,
                                     dtype=torch.float16)
            setattr(parent, name, shell)


# An fp16 rotation multiplies activations (typically |x| < 100) by the channel scale: above this bound the
# product can leave the fp16 range (65504) and turn into inf, then NaN.
_FP16_SAFE_SCALE = 65504.0 / 128.0


def _sanitise_channel_scales(model):
    """Clip every RotateLinearInt4's channel scales to +-65504/128 in place (inf included) and report the
    modules touched (paroquant_marlin_w4a8.py:390-423).  As in the reference, the clip leaves NaN entries
    NaN; they are reported separately because no clip can repair them.  Returns the number of modules whose
    scales were out of range."""
    touched = 0
    for name, rl in model.named_modules():
        if not isinstance(rl, RotateLinearInt4):
            continue
        cs = rl.rotation.channel_scales
        nan = torch.isnan(cs)
        out_of_range = torch.isinf(cs) | (cs.abs() > _FP16_SAFE_SCALE)
        n_nan, n_big = int(nan.sum()), int(out_of_range.sum())
        if n_nan + n_big == 0:
            continue
        touched += 1
        with torch.no_grad():
            cs.clamp_(min=-_FP16_SAFE_SCALE, max=_FP16_SAFE_SCALE)
        logger.warning("%s: %d of %d channel scales beyond +-%.0f (or infinite) clipped; %d NaN left as they are",
                       name, n_big, cs.numel(), _FP16_SAFE_SCALE, n_nan)
    if touched:
        logger.warning("channel scales clipped in %d RotateLinearInt4 module(s)", touched)
    else:
        logger.info("channel scales: every value within the fp16-safe range")
    return touched


class LoadReport(NamedTuple):
    """What load_paroquant_checkpoint found (the reference logs the same diagnostics,
    paroquant_marlin_w4a8.py:466-502)."""
    missing: list            # model keys the checkpoint lacks
    unexpected: list         # checkpoint keys the model lacks
    quant_missing: list      # missing keys of quantized modules (rotation / qlinear buffers)
    zero_scales: list        # names of non-empty "scales" tensors that are all zero after loading
    sanitised: int           # modules whose channel scales were clipped


_QUANT_KEY_PARTS = ("qlinear", "rotation", "qweight", "scales", "scaled_zeros")


def _all_zero_scale_tensors(model) -> list:
    """Names of non-empty parameters or buffers with "scales" in their name that hold only zeros: a
    quantized layer whose checkpoint entries did not load (its outputs would be all zero)."""
    named = list(model.named_parameters()) + list(model.named_buffers())
    return [n for n, t in named if "scales" in n and t.numel() > 0 and not bool(t.detach().ne(0).any())]


def load_paroquant_checkpoint(model, paro_checkpoint, *, target="vlm", device="cuda", wrap_bf16=True):
    """Load a ParoQuant state dict into an already-built model: the checkpoint half of the reference's
    load_paroquant_model (paroquant_marlin_w4a8.py:426-510), whose first half builds the AlpamayoR1 model.

    Replaces the target layers' linears by RotateLinearInt4 shells, reads the state dict
    (``torch.load(..., weights_only=True)`` for a path; a dict is used as is), loads it non-strictly, reports
    key overlap, missing and unexpected keys and quantized layers whose scales stayed all zero, clips
    out-of-range channel scales, wraps the shells for bf16 activations, and moves the model to `device` in
    eval mode.  Returns (model, LoadReport).
    """
    replace_linears_with_rotate_linear(model, target=target, init_only=True)
    if isinstance(paro_checkpoint, (str, bytes)) or hasattr(paro_checkpoint, "__fspath__"):
        state = torch.load(paro_checkpoint, map_location="cpu", weights_only=True)
    else:
        state = paro_checkpoint
    have, given = set(model.state_dict()), set(state)
    logger.info("ParoQuant checkpoint: %d tensors, model: %d, shared: %d", len(given), len(have), len(have & given))
    missing, unexpected = model.load_state_dict(state, strict=False)
    quant_missing = [k for k in missing if any(part in k for part in _QUANT_KEY_PARTS)]
    if quant_missing:
        logger.warning("%d missing keys, %d of them quantization buffers, e.g. %s", len(missing),
                       len(quant_missing), quant_missing[:10])
    elif missing:
        logger.info("%d missing keys (no quantization buffer among them), e.g. %s", len(missing), missing[:5])
    if unexpected:
        logger.warning("%d checkpoint keys the model does not have, e.g. %s", len(unexpected), unexpected[:20])
    del state
    zero = _all_zero_scale_tensors(model)
    if zero:
        logger.error("%d quantized scale tensors are all zero after loading (checkpoint keys probably do not "
                     "match the model), e.g. %s", len(zero), zero[:3])
    else:
        logger.info("every quantized scale tensor holds non-zero values")
    fixed = _sanitise_channel_scales(model)
    if wrap_bf16:
        _wrap_rotate_linears(model, target=target)
    model.to(device)
    model.eval()
    return model, LoadReport(list(missing), list(unexpected), quant_missing, zero, fixed)


def convert_model_to_marlin_w4a8(model):
    """Give every RotateLinearInt4 that holds a WQLinear a MarlinW4A8Linear with the same weights, on the
    WQLinear's device, and derive its rotation's packed operands; returns how many were converted
    (paroquant_marlin_w4a8.py:513-529)."""
    todo = [rl for rl in model.modules() if isinstance(rl, RotateLinearInt4) and isinstance(rl.qlinear, WQLinear)]
    for rl in todo:
        wq = rl.qlinear
        rl.qlinear, _ = convert_wqlinear_layer(wq.qweight.data, wq.scales.data, wq.scaled_zeros.data,
                                               wq.out_features, wq.in_features, wq.group_size, bias=wq.bias,
                                               device=wq.qweight.device)
        rl.rotation.prepare()
    logger.info("%d RotateLinearInt4 layer(s) now run the W4A8 kernels", len(todo))
    return len(todo)
