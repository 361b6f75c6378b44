"""torch custom ops over libparoquant_hip.so.

``torch.ops.rotation.rotate`` has the reference's exact schema
(kernels/paroquant_kernels/src/rotation.cu:576-579); the other ops live in
the ``paroquant`` namespace:

  rotation::rotate(x, idx_ij, theta, scales?, group_size) -> y
  paroquant::rotate_backward(grad_y, x, idx_ij, theta, scales?, group_size) -> (grad_x, grad_theta, grad_scales)
  paroquant::rotate_quant_i8(x, rot_idx, rot_cs, scales?, krot, input_fp16, materialize_fp16) -> (xq, xscale)
  paroquant::rotate_quant_i8_rot(...)                 -> (xq, xscale, xrot fp16)
  paroquant::quant_i8(x) -> (xq, xscale)
  paroquant::w4a8_gemm(xq, xscale, wpack, wmeta, bias?, out_dtype) -> y
  paroquant::w4a8_gemm_partials(xq, wpack, wmeta) -> int32 [m, k/128, n]
  paroquant::w4a8_prepack(awq_qweight, awq_scales, awq_qzeros) -> (wpack, wmeta)
  paroquant::w4a8_linear(x, rot_idx, rot_cs, scales?, krot, wpack, wmeta, bias?,
                         input_fp16, materialize_fp16, out_dtype) -> y
  paroquant::w4a8_linear_group(x, rot_idx[], rot_cs[], scales?[], krot, wpack[], wmeta[], bias?[],
                               input_fp16, materialize_fp16, out_dtype) -> y[]
      (1..4 linears sharing the input x, in two launches for the whole group)
  paroquant::w4a8_linear_group_rmsnorm(x, residual?, norm_weight, eps, <the group's arguments>,
                                       return_normed, return_sum) -> y[] (+ h) (+ x + residual)
      (the same group behind a decoder layer's RMSNorm of x + residual, still two launches)

``pack_rotation`` (host) turns Rotation's pairs/angles into rot_idx/rot_cs;
``register_packed_rotation`` lets rotation::rotate find them (it never packs
them itself).

Implementations are registered for the CUDA (HIP) dispatch key only, like the
reference (rotation.cu:581-584); CPU tensors raise from the dispatcher.  Each
op has a fake (meta) kernel so torch.compile and graph capture can trace it.
Every op allocates its outputs with torch on the input's device and enqueues
its kernels on the current stream; none synchronises.  Scratch between an
op's kernels comes from torch's caching allocator (inside a graph capture,
the graph's pool at fixed addresses); the C ABI below takes it as an
explicit workspace argument instead.
"""

from __future__ import annotations

import weakref
from collections import OrderedDict

import torch

from . import _lib

_DT = {torch.float32: _lib.PQ_F32, torch.float16: _lib.PQ_F16, torch.bfloat16: _lib.PQ_BF16}

_rotation_lib = torch.library.Library("rotation", "DEF")
_rotation_lib.define("rotate(Tensor x, Tensor idx_ij, Tensor theta, Tensor? scales, int group_size) -> Tensor")
# The reference's rotate_and_quant writes NVFP4; this is the same fused op in the OCP MXFP4 format
# (codes uint8 [..., H/2], E8M0 scales uint8 [..., H/32]).
_rotation_lib.define("rotate_and_quant_mxfp4(Tensor x, Tensor idx_ij, Tensor theta, Tensor? scales, "
                     "int group_size) -> (Tensor, Tensor)")

_pq_lib = torch.library.Library("paroquant", "DEF")
# Gradients of rotation::rotate (grad_x, grad_theta, grad_scales; the last empty when scales is None).
_pq_lib.define("rotate_backward(Tensor grad_y, Tensor x, Tensor idx_ij, Tensor theta, Tensor? scales, "
               "int group_size) -> (Tensor, Tensor, Tensor)")
_pq_lib.define("rotate_quant_i8(Tensor x, Tensor rot_idx, Tensor rot_cs, Tensor? scales, int krot, bool input_fp16, "
               "bool materialize_fp16) -> (Tensor, Tensor)")
_pq_lib.define("rotate_quant_i8_rot(Tensor x, Tensor rot_idx, Tensor rot_cs, Tensor? scales, int krot, "
               "bool input_fp16, bool materialize_fp16) -> (Tensor, Tensor, Tensor)")
_pq_lib.define("quant_i8(Tensor x) -> (Tensor, Tensor)")
_pq_lib.define("w4a8_gemm(Tensor xq, Tensor xscale, Tensor wpack, Tensor wmeta, Tensor? bias, "
               "ScalarType out_dtype) -> Tensor")
_pq_lib.define("w4a8_gemm_partials(Tensor xq, Tensor wpack, Tensor wmeta) -> Tensor")
_pq_lib.define("w4a8_prepack(Tensor awq_qweight, Tensor awq_scales, Tensor awq_qzeros) -> (Tensor, Tensor)")
_pq_lib.define("w4a8_linear(Tensor x, Tensor rot_idx, Tensor rot_cs, Tensor? scales, int krot, Tensor wpack, "
               "Tensor wmeta, Tensor? bias, bool input_fp16, bool materialize_fp16, "
               "ScalarType out_dtype) -> Tensor")
_pq_lib.define("w4a8_linear_group(Tensor x, Tensor[] rot_idx, Tensor[] rot_cs, Tensor?[] scales, int krot, "
               "Tensor[] wpack, Tensor[] wmeta, Tensor?[] bias, bool input_fp16, "
               "bool materialize_fp16, ScalarType out_dtype) -> Tensor[]")
_pq_lib.define("w4a8_linear_group_rmsnorm(Tensor x, Tensor? residual, Tensor norm_weight, float eps, "
               "Tensor[] rot_idx, Tensor[] rot_cs, Tensor?[] scales, int krot, Tensor[] wpack, Tensor[] wmeta, "
               "Tensor?[] bias, bool input_fp16, bool materialize_fp16, ScalarType out_dtype, "
               "bool return_normed, bool return_sum) -> Tensor[]")
_pq_lib.define("w4a8_linear_group_fused(Tensor x, Tensor? x2, Tensor? norm_weight, float eps, int mode, "
               "Tensor[] rot_idx, Tensor[] rot_cs, Tensor?[] scales, int krot, Tensor[] wpack, Tensor[] wmeta, "
               "Tensor?[] bias, bool input_fp16, bool materialize_fp16, ScalarType out_dtype, "
               "bool return_h, bool return_sum) -> Tensor[]")
_pq_lib.define("w4a16_prepack(Tensor awq_qweight, Tensor scales, Tensor scaled_zeros) -> (Tensor, Tensor)")
_pq_lib.define("w4a16_gemm(Tensor x, Tensor wpack, Tensor wmeta, Tensor? bias, ScalarType out_dtype) -> Tensor")
_pq_lib.define("w4a16_linear_group(Tensor x, Tensor[] rot_idx, Tensor[] rot_cs, Tensor?[] scales, int krot, "
               "Tensor[] wpack, Tensor[] wmeta, Tensor?[] bias, bool input_fp16, "
               "ScalarType out_dtype) -> Tensor[]")
_pq_lib.define("w4a16_linear(Tensor x, Tensor rot_idx, Tensor rot_cs, Tensor? scales, int krot, Tensor wpack, "
               "Tensor wmeta, Tensor? bias, bool input_fp16, ScalarType out_dtype) -> Tensor")


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------

def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


class _DeviceGuard:
    """Makes `dev` current for the duration of a call when it is not already."""

    __slots__ = ("dev", "prev")

    def __init__(self, dev: torch.device):
        self.dev = dev
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if self.dev.index is not None and self.dev.index != cur:
            self.prev = cur
            torch.cuda.set_device(self.dev)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _same_device(name: str, t: torch.Tensor, dev: torch.device) -> None:
    _require(t.device == dev, f"{name}: expected a tensor on {dev}, got {t.device}")


def gemm_dims(wpack: torch.Tensor) -> tuple[int, int]:
    """(out_features, in_features) of a prepacked weight [N/16, K/128, 64, 16]."""
    _require(wpack.dim() == 4 and wpack.size(2) == 64 and wpack.size(3) == 16 and wpack.dtype == torch.uint8,
             "wpack must be uint8 [N/16, K/128, 64, 16]")
    return wpack.size(0) * 16, wpack.size(1) * 128


def workspace_bytes(m: int, n: int, k: int) -> int:
    return int(_lib.load().pq_w4a8_workspace_size(m, n, k, 128))


def linear_workspace_bytes(m: int, n: int, k: int, krot: int) -> int:
    """Scratch bytes paroquant::w4a8_linear needs between its two kernels for m tokens."""
    return int(_lib.load().pq_w4a8_linear_workspace_size(m, n, k, krot))


# ---------------------------------------------------------------------------
# rotation::rotate
# ---------------------------------------------------------------------------

def _rotate_args(x, idx_ij, theta, scales):
    """Checks of rotation::rotate's arguments; contiguous copies and the sizes."""
    _require(x.dtype in _DT, f"rotate only supports Float, Half, and BFloat16, but got {x.dtype}")
    _require(idx_ij.dtype == torch.int16, f"idx_ij must be int16, got {idx_ij.dtype}")
    _require(theta.dtype == x.dtype, f"theta must have x's dtype {x.dtype}, got {theta.dtype}")
    _require(x.dim() >= 1 and x.size(-1) > 0, "x must have a non-empty last dimension")
    h = x.size(-1)
    _require(idx_ij.dim() == 2 and theta.dim() == 2, "idx_ij and theta must be 2-D [KROT, H] / [KROT, H/2]")
    krot = theta.size(0)
    _require(krot == idx_ij.size(0), "theta.size(0) must equal idx_ij.size(0)")
    _require(idx_ij.size(1) == h and theta.size(1) * 2 == h,
             f"idx_ij must be [KROT, {h}] and theta [KROT, {h // 2}], got {tuple(idx_ij.shape)} / {tuple(theta.shape)}")
    has_scale = scales is not None and scales.numel() > 0
    if has_scale:
        _require(scales.dtype == x.dtype, f"scales must have x's dtype {x.dtype}, got {scales.dtype}")
        _require(scales.numel() == h, f"scales must hold {h} values, got {scales.numel()}")
    dev = x.device
    for nm, t in (("idx_ij", idx_ij), ("theta", theta)) + ((("scales", scales),) if has_scale else ()):
        _same_device(nm, t, dev)
    xc = x.contiguous()
    scc = scales.contiguous() if has_scale else None
    return xc, idx_ij.contiguous(), theta.contiguous(), scc, xc.numel() // h, h, krot


# Packed operands of rotation::rotate's (pairs, angles, scales), registered by whoever derived them
# (Rotation.prepare()): the register-chain kernel of the fused linear runs whole rows about 1.5x faster than
# the LDS-tile kernel at large row counts, and gives the same results (both take cos/sin of each angle in
# float64, rounded once).  The op itself only looks them up -- it never packs, copies to the host or
# synchronizes -- and runs the tile kernel, which derives its parameters on the device, when nothing
# current is registered for its exact tensors.
_PACK_REGISTRY: "OrderedDict" = OrderedDict()
_PACK_REGISTRY_MAX = 4096
_PACKED_MIN_ROWS = 1024


def _none_ref():
    return None


def tensor_state(t: torch.Tensor | None):
    """(data pointer, in-place version, device) of t: it changes whenever t is modified in place or replaced.
    Tensors made under torch.inference_mode() carry no version counter; their pointer and device stand in."""
    if t is None:
        return None
    try:
        ver = t._version
    except RuntimeError:
        ver = None
    return (t.data_ptr(), ver, t.device)


def _tensor_state(srcs):
    return tuple(tensor_state(t) for t in srcs)


def register_packed_rotation(idx_ij, theta, scales, rot_idx, rot_cs, scales_f32) -> None:
    """Records (rot_idx, rot_cs, scales_f32), derived from exactly these (idx_ij, theta, scales) tensors, for
    rotation::rotate and rotation::rotate_and_quant_mxfp4 on those tensors.  The entry lapses as soon as any of
    the three tensors is modified in place, freed, or replaced."""
    srcs = (idx_ij, theta, scales)
    key = tuple(id(t) for t in srcs)
    refs = tuple(weakref.ref(t) if t is not None else _none_ref for t in srcs)
    _PACK_REGISTRY[key] = (refs, _tensor_state(srcs), (rot_idx, rot_cs, scales_f32))
    _PACK_REGISTRY.move_to_end(key)
    while len(_PACK_REGISTRY) > _PACK_REGISTRY_MAX:
        _PACK_REGISTRY.popitem(last=False)


def _packed_for(idx_ij, theta, scales, group_size):
    """The registered (rot_idx, rot_cs, scales_f32) of these tensors, or None: nothing registered, a stale
    entry, group 64, angles that require grad (trained: they change every step), or tensors made under
    torch.inference_mode(), which carry no version counter, so an in-place change to them could not be seen
    (the op then derives its parameters on the device: same results)."""
    if group_size != 128 or theta.requires_grad:
        return None
    srcs = (idx_ij, theta, scales)
    ent = _PACK_REGISTRY.get(tuple(id(t) for t in srcs))
    if ent is None:
        return None
    refs, state, packed = ent
    now = _tensor_state(srcs)
    if any(st is not None and st[1] is None for st in now):
        return None
    if state != now or not all(r() is t for r, t in zip(refs, srcs)):
        return None
    if packed[0].device != idx_ij.device:
        return None
    return packed


def _rotate_rows(xc, packed, out, mx_scales, rows, h, krot, mode, what):
    rot_idx, rot_cs, sf = packed
    lib = _lib.load()
    with _DeviceGuard(xc.device):
        st = lib.pq_rotate_rows(xc.data_ptr(), _DT[xc.dtype], rot_idx.data_ptr(), rot_cs.data_ptr(),
                                sf.data_ptr() if sf is not None else None, out.data_ptr(),
                                mx_scales.data_ptr() if mx_scales is not None else None, rows, h, krot, mode,
                                _stream(xc.device))
    _lib.check(st, what)


def _rotate_impl(x, idx_ij, theta, scales, group_size):
    xc, idc, thc, scc, rows, h, krot = _rotate_args(x, idx_ij, theta, scales)
    dev = x.device
    out = torch.empty_like(xc)
    if rows >= _PACKED_MIN_ROWS:
        packed = _packed_for(idx_ij, theta, scales if scc is not None else None, group_size)
        if packed is not None:
            _rotate_rows(xc, packed, out, None, rows, h, krot, _lib.PQ_ROWS_SAME, "rotation::rotate")
            return out
    lib = _lib.load()
    with _DeviceGuard(dev):
        st = lib.pq_rotate(xc.data_ptr(), out.data_ptr(), idc.data_ptr(), thc.data_ptr(),
                           scc.data_ptr() if scc is not None else None, rows, h, krot, int(group_size),
                           _DT[x.dtype], _stream(dev))
    _lib.check(st, "rotation::rotate")
    return out


def _rotate_mxfp4_impl(x, idx_ij, theta, scales, group_size):
    xc, idc, thc, scc, rows, h, krot = _rotate_args(x, idx_ij, theta, scales)
    _require(h % 32 == 0, f"MXFP4 blocks are 32 channels: h={h}")
    dev = x.device
    q = torch.empty((*x.shape[:-1], h // 2), dtype=torch.uint8, device=dev)
    sc = torch.empty((*x.shape[:-1], h // 32), dtype=torch.uint8, device=dev)
    if rows >= _PACKED_MIN_ROWS:
        packed = _packed_for(idx_ij, theta, scales if scc is not None else None, group_size)
        if packed is not None:
            _rotate_rows(xc, packed, q, sc, rows, h, krot, _lib.PQ_ROWS_MXFP4, "rotation::rotate_and_quant_mxfp4")
            return q, sc
    lib = _lib.load()
    with _DeviceGuard(dev):
        st = lib.pq_rotate_mxfp4(xc.data_ptr(), q.data_ptr(), sc.data_ptr(), idc.data_ptr(), thc.data_ptr(),
                                 scc.data_ptr() if scc is not None else None, rows, h, krot, int(group_size),
                                 _DT[x.dtype], _stream(dev))
    _lib.check(st, "rotation::rotate_and_quant_mxfp4")
    return q, sc


_rotation_lib.impl("rotate", _rotate_impl, "CUDA")


@torch.library.register_fake("rotation::rotate")
def _rotate_fake(x, idx_ij, theta, scales, group_size):
    return x.new_empty(x.shape)


_rotation_lib.impl("rotate_and_quant_mxfp4", _rotate_mxfp4_impl, "CUDA")


@torch.library.register_fake("rotation::rotate_and_quant_mxfp4")
def _rotate_mxfp4_fake(x, idx_ij, theta, scales, group_size):
    h = x.size(-1)
    return (x.new_empty((*x.shape[:-1], h // 2), dtype=torch.uint8),
            x.new_empty((*x.shape[:-1], h // 32), dtype=torch.uint8))


def _rotate_backward_impl(grad_y, x, idx_ij, theta, scales, group_size):
    xc, idc, thc, scc, rows, h, krot = _rotate_args(x, idx_ij, theta, scales)
    _require(grad_y.shape == x.shape and grad_y.dtype == x.dtype,
             f"grad_y must match x ({tuple(x.shape)}, {x.dtype}), got {tuple(grad_y.shape)}, {grad_y.dtype}")
    dev = x.device
    _same_device("grad_y", grad_y, dev)
    gyc = grad_y.contiguous()
    gx = torch.empty_like(xc)
    gth = torch.empty_like(thc)
    gs = torch.empty_like(scc) if scc is not None else x.new_empty((0,))
    lib = _lib.load()
    need = int(lib.pq_rotate_backward_workspace_size(rows, h, krot))
    ws = torch.empty(need, dtype=torch.uint8, device=dev) if need else None
    with _DeviceGuard(dev):
        st = lib.pq_rotate_backward(xc.data_ptr(), gyc.data_ptr(), gx.data_ptr(), gth.data_ptr(),
                                    gs.data_ptr() if scc is not None else None, idc.data_ptr(), thc.data_ptr(),
                                    scc.data_ptr() if scc is not None else None, rows, h, krot, int(group_size),
                                    _DT[x.dtype], ws.data_ptr() if ws is not None else None, need, _stream(dev))
    _lib.check(st, "paroquant::rotate_backward")
    return gx.view(x.shape), gth.view(theta.shape), gs.view(scales.shape) if scc is not None else gs


_pq_lib.impl("rotate_backward", _rotate_backward_impl, "CUDA")


@torch.library.register_fake("paroquant::rotate_backward")
def _rotate_backward_fake(grad_y, x, idx_ij, theta, scales, group_size):
    has_scale = scales is not None and scales.numel() > 0
    return (x.new_empty(x.shape), theta.new_empty(theta.shape),
            scales.new_empty(scales.shape) if has_scale else x.new_empty((0,)))


# ---------------------------------------------------------------------------
# paroquant::rotate_quant_i8 / rotate_quant_i8_rot / quant_i8
# ---------------------------------------------------------------------------

def packed_rotation_shapes(h: int, krot: int) -> tuple[tuple, tuple]:
    kp = 8 if krot <= 8 else 16
    return (h // 128, 64, kp // 2), (h // 128, 64, kp, 2)


def pack_rotation(pairs: torch.Tensor, cos_sin: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Host packing of pairs int16 [krot, h] and cos_sin float32 [krot, h/2, 2] into
    (rot_idx int32 [h/128, 64, KP/2], rot_cs float32 [h/128, 64, KP, 2]) on the CPU,
    KP = 8 for krot <= 8 else 16.  Raises ValueError unless every layer pairs each
    channel of each 128-group exactly once."""
    p = pairs.detach().to("cpu", torch.int16).contiguous()
    cs = cos_sin.detach().to("cpu", torch.float32).contiguous()
    krot, h = p.shape
    _require(tuple(cs.shape) == (krot, h // 2, 2), f"cos_sin must be [{krot}, {h // 2}, 2]")
    sij, scs = packed_rotation_shapes(h, krot)
    rot_idx = torch.empty(sij, dtype=torch.int32)
    rot_cs = torch.empty(scs, dtype=torch.float32)
    st = _lib.load().pq_rotation_pack(p.data_ptr(), cs.data_ptr(), h, krot, rot_idx.data_ptr(), rot_cs.data_ptr())
    if st == _lib.STATUS_CODE["PQ_ERR_ARG"]:
        raise ValueError(_lib.load().pq_last_error().decode())
    _lib.check(st, "pack_rotation")
    return rot_idx, rot_cs


def _check_rot_params(x, rot_idx, rot_cs, scales, krot):
    h = x.size(-1)
    _require(x.dtype in _DT, f"x must be float32/float16/bfloat16, got {x.dtype}")
    _require(h % 128 == 0 and 0 < h <= 16384, f"in_features={h} must be a multiple of 128 and <= 16384")
    _require(1 <= krot <= 16, f"KROT={krot} must be in 1..16")
    sij, scs = packed_rotation_shapes(h, krot)
    _require(rot_idx.dtype in (torch.int32, torch.uint32) and tuple(rot_idx.shape) == sij,
             f"rot_idx must be int32 {sij}, got {rot_idx.dtype} {tuple(rot_idx.shape)}")
    _require(rot_cs.dtype == torch.float32 and tuple(rot_cs.shape) == scs,
             f"rot_cs must be float32 {scs}, got {rot_cs.dtype} {tuple(rot_cs.shape)}")
    if scales is not None:
        _require(scales.dtype == torch.float32 and scales.numel() == h,
                 f"scales must be float32 with {h} values, got {scales.dtype} {scales.numel()}")
    dev = x.device
    _same_device("rot_idx", rot_idx, dev)
    _same_device("rot_cs", rot_cs, dev)
    if scales is not None:
        _same_device("scales", scales, dev)
    return h


def _rotate_quant(x, rot_idx, rot_cs, scales, krot, input_fp16, materialize_fp16, want_rot):
    h = _check_rot_params(x, rot_idx, rot_cs, scales, krot)
    dev = x.device
    xc = x.contiguous()
    rows = xc.numel() // h
    xq = torch.empty((rows, h), dtype=torch.int8, device=dev)
    xs = torch.empty((rows,), dtype=torch.float32, device=dev)
    xr = torch.empty((rows, h), dtype=torch.float16, device=dev) if want_rot else None
    flags = (_lib.PQ_RQ_INPUT_FP16 if input_fp16 else 0) | (_lib.PQ_RQ_MATERIALIZE_FP16 if materialize_fp16 else 0)
    idx, cs = rot_idx.contiguous(), rot_cs.contiguous()
    sc = scales.contiguous() if scales is not None else None
    lib = _lib.load()
    with _DeviceGuard(dev):
        st = lib.pq_rotate_quant_i8(xc.data_ptr(), _DT[x.dtype], idx.data_ptr(), cs.data_ptr(),
                                    sc.data_ptr() if sc is not None else None, xq.data_ptr(), xs.data_ptr(),
                                    xr.data_ptr() if xr is not None else None, rows, h, krot, flags, _stream(dev))
    _lib.check(st, "paroquant::rotate_quant_i8")
    return xq, xs, xr


def _rotate_quant_impl(x, rot_idx, rot_cs, scales, krot, input_fp16, materialize_fp16):
    xq, xs, _ = _rotate_quant(x, rot_idx, rot_cs, scales, krot, input_fp16, materialize_fp16, False)
    return xq, xs


def _rotate_quant_rot_impl(x, rot_idx, rot_cs, scales, krot, input_fp16, materialize_fp16):
    return _rotate_quant(x, rot_idx, rot_cs, scales, krot, input_fp16, materialize_fp16, True)


_pq_lib.impl("rotate_quant_i8", _rotate_quant_impl, "CUDA")
_pq_lib.impl("rotate_quant_i8_rot", _rotate_quant_rot_impl, "CUDA")


@torch.library.register_fake("paroquant::rotate_quant_i8")
def _rotate_quant_fake(x, rot_idx, rot_cs, scales, krot, input_fp16, materialize_fp16):
    h = x.size(-1)
    rows = x.numel() // h
    return (x.new_empty((rows, h), dtype=torch.int8), x.new_empty((rows,), dtype=torch.float32))


@torch.library.register_fake("paroquant::rotate_quant_i8_rot")
def _rotate_quant_rot_fake(x, rot_idx, rot_cs, scales, krot, input_fp16, materialize_fp16):
    h = x.size(-1)
    rows = x.numel() // h
    return (x.new_empty((rows, h), dtype=torch.int8), x.new_empty((rows,), dtype=torch.float32),
            x.new_empty((rows, h), dtype=torch.float16))


def _quant_impl(x):
    _require(x.dtype in _DT, f"x must be float32/float16/bfloat16, got {x.dtype}")
    h = x.size(-1)
    _require(h % 8 == 0 and h > 0, f"last dimension {h} must be a positive multiple of 8")
    dev = x.device
    xc = x.contiguous()
    rows = xc.numel() // h
    xq = torch.empty((rows, h), dtype=torch.int8, device=dev)
    xs = torch.empty((rows,), dtype=torch.float32, device=dev)
    lib = _lib.load()
    with _DeviceGuard(dev):
        st = lib.pq_quant_i8(xc.data_ptr(), _DT[x.dtype], xq.data_ptr(), xs.data_ptr(), rows, h, _stream(dev))
    _lib.check(st, "paroquant::quant_i8")
    return xq, xs


_pq_lib.impl("quant_i8", _quant_impl, "CUDA")


@torch.library.register_fake("paroquant::quant_i8")
def _quant_fake(x):
    h = x.size(-1)
    rows = x.numel() // h
    return x.new_empty((rows, h), dtype=torch.int8), x.new_empty((rows,), dtype=torch.float32)


# ---------------------------------------------------------------------------
# paroquant::w4a8_gemm / w4a8_gemm_partials / w4a8_prepack / w4a8_linear
# ---------------------------------------------------------------------------

def _check_weights(wpack, wmeta, dev):
    n, k = gemm_dims(wpack)
    _require(wmeta.dtype in (torch.int32, torch.uint32) and tuple(wmeta.shape) == (n // 16, k // 128, 16),
             f"wmeta must be int32 [{n // 16}, {k // 128}, 16], got {wmeta.dtype} {tuple(wmeta.shape)}")
    _require(wpack.is_contiguous() and wmeta.is_contiguous(), "wpack/wmeta must be contiguous")
    _same_device("wpack", wpack, dev)
    _same_device("wmeta", wmeta, dev)
    return n, k


def _gemm_launch(xq, xs, wpack, wmeta, bias, out_dtype, m, n, k, dev):
    _require(out_dtype in _DT, f"out_dtype must be float32/float16/bfloat16, got {out_dtype}")
    y = torch.empty((m, n), dtype=out_dtype, device=dev)
    if bias is not None:
        _require(bias.dtype in _DT and bias.numel() == n, f"bias must hold {n} float values")
        _same_device("bias", bias, dev)
        bias = bias.contiguous()
    need = workspace_bytes(m, n, k)
    ws_ptr, ws_bytes = None, 0
    if need > 0:
        workspace = torch.zeros(need, dtype=torch.uint8, device=dev)
        ws_ptr, ws_bytes = workspace.data_ptr(), need
    lib = _lib.load()
    with _DeviceGuard(dev):
        st = lib.pq_w4a8_gemm(xq.data_ptr(), xs.data_ptr(), wpack.data_ptr(), wmeta.data_ptr(),
                              bias.data_ptr() if bias is not None else None,
                              _DT[bias.dtype] if bias is not None else 0, y.data_ptr(), _DT[out_dtype], m, n, k, 128,
                              ws_ptr, ws_bytes, _stream(dev))
    _lib.check(st, "paroquant::w4a8_gemm")
    return y


def _gemm_impl(xq, xscale, wpack, wmeta, bias, out_dtype):
    dev = xq.device
    n, k = _check_weights(wpack, wmeta, dev)
    _require(xq.dtype == torch.int8 and xq.dim() == 2 and xq.size(1) == k,
             f"xq must be int8 [M, {k}], got {xq.dtype} {tuple(xq.shape)}")
    m = xq.size(0)
    _require(xscale.dtype == torch.float32 and xscale.numel() == m, f"xscale must be float32 [{m}]")
    _same_device("xscale", xscale, dev)
    return _gemm_launch(xq.contiguous(), xscale.contiguous(), wpack, wmeta, bias, out_dtype, m, n, k, dev)


_pq_lib.impl("w4a8_gemm", _gemm_impl, "CUDA")


@torch.library.register_fake("paroquant::w4a8_gemm")
def _gemm_fake(xq, xscale, wpack, wmeta, bias, out_dtype):
    return xq.new_empty((xq.size(0), wpack.size(0) * 16), dtype=out_dtype)


def _partials_impl(xq, wpack, wmeta):
    dev = xq.device
    n, k = _check_weights(wpack, wmeta, dev)
    _require(xq.dtype == torch.int8 and xq.dim() == 2 and xq.size(1) == k, f"xq must be int8 [M, {k}]")
    m = xq.size(0)
    out = torch.empty((m, k // 128, n), dtype=torch.int32, device=dev)
    xc = xq.contiguous()
    lib = _lib.load()
    with _DeviceGuard(dev):
        st = lib.pq_w4a8_gemm_partials(xc.data_ptr(), wpack.data_ptr(), wmeta.data_ptr(), out.data_ptr(), m, n, k,
                                       128, _stream(dev))
    _lib.check(st, "paroquant::w4a8_gemm_partials")
    return out


_pq_lib.impl("w4a8_gemm_partials", _partials_impl, "CUDA")


@torch.library.register_fake("paroquant::w4a8_gemm_partials")
def _partials_fake(xq, wpack, wmeta):
    return xq.new_empty((xq.size(0), wpack.size(1), wpack.size(0) * 16), dtype=torch.int32)


def _prepack_impl(awq_qweight, awq_scales, awq_qzeros):
    dev = awq_qweight.device
    _require(awq_qweight.dtype == torch.int32 and awq_qweight.dim() == 2, "awq_qweight must be int32 [K, N/8]")
    k, n = awq_qweight.size(0), awq_qweight.size(1) * 8
    _require(k % 128 == 0 and n % 16 == 0, f"K={k} must be a multiple of 128 and N={n} of 16")
    g = k // 128
    _require(awq_scales.dtype == torch.float16 and tuple(awq_scales.shape) == (g, n),
             f"awq_scales must be float16 [{g}, {n}], got {awq_scales.dtype} {tuple(awq_scales.shape)}")
    _require(awq_qzeros.dtype == torch.int32 and tuple(awq_qzeros.shape) == (g, n // 8),
             f"awq_qzeros must be int32 [{g}, {n // 8}], got {awq_qzeros.dtype} {tuple(awq_qzeros.shape)}")
    _same_device("awq_scales", awq_scales, dev)
    _same_device("awq_qzeros", awq_qzeros, dev)
    qw, sc, qz = awq_qweight.contiguous(), awq_scales.contiguous(), awq_qzeros.contiguous()
    wpack = torch.empty((n // 16, g, 64, 16), dtype=torch.uint8, device=dev)
    wmeta = torch.empty((n // 16, g, 16), dtype=torch.int32, device=dev)
    lib = _lib.load()
    with _DeviceGuard(dev):
        st = lib.pq_w4a8_prepack(qw.data_ptr(), sc.data_ptr(), qz.data_ptr(), wpack.data_ptr(), wmeta.data_ptr(), k,
                                 n, 128, _stream(dev))
    _lib.check(st, "paroquant::w4a8_prepack")
    return wpack, wmeta


_pq_lib.impl("w4a8_prepack", _prepack_impl, "CUDA")


@torch.library.register_fake("paroquant::w4a8_prepack")
def _prepack_fake(awq_qweight, awq_scales, awq_qzeros):
    k, n = awq_qweight.size(0), awq_qweight.size(1) * 8
    return (awq_qweight.new_empty((n // 16, k // 128, 64, 16), dtype=torch.uint8),
            awq_qweight.new_empty((n // 16, k // 128, 16), dtype=torch.int32))


def _linear_impl(x, rot_idx, rot_cs, scales, krot, wpack, wmeta, bias, input_fp16, materialize_fp16, out_dtype):
    dev = x.device
    n, k = _check_weights(wpack, wmeta, dev)
    _require(x.size(-1) == k, f"x has {x.size(-1)} features, the weights expect {k}")
    _check_rot_params(x, rot_idx, rot_cs, scales, krot)
    _require(out_dtype in _DT, f"out_dtype must be float32/float16/bfloat16, got {out_dtype}")
    xc = x.contiguous()
    m = xc.numel() // k
    y = torch.empty((m, n), dtype=out_dtype, device=dev)
    if bias is not None:
        _require(bias.dtype in _DT and bias.numel() == n, f"bias must hold {n} float values")
        _same_device("bias", bias, dev)
        bias = bias.contiguous()
    lib = _lib.load()
    need = int(lib.pq_w4a8_linear_workspace_size(m, n, k, krot))
    scratch = torch.empty(need, dtype=torch.uint8, device=dev) if need > 0 else None
    flags = (_lib.PQ_RQ_INPUT_FP16 if input_fp16 else 0) | (_lib.PQ_RQ_MATERIALIZE_FP16 if materialize_fp16 else 0)
    idx, cs = rot_idx.contiguous(), rot_cs.contiguous()
    sc = scales.contiguous() if scales is not None else None
    with _DeviceGuard(dev):
        st = lib.pq_w4a8_linear(xc.data_ptr(), _DT[x.dtype], idx.data_ptr(), cs.data_ptr(),
                                sc.data_ptr() if sc is not None else None, wpack.data_ptr(), wmeta.data_ptr(),
                                bias.data_ptr() if bias is not None else None,
                                _DT[bias.dtype] if bias is not None else 0, y.data_ptr(), _DT[out_dtype], m, n, k,
                                krot, flags, scratch.data_ptr() if scratch is not None else None,
                                scratch.numel() if scratch is not None else 0,
                                _stream(dev))
    _lib.check(st, "paroquant::w4a8_linear")
    return y.view(*x.shape[:-1], n)


_pq_lib.impl("w4a8_linear", _linear_impl, "CUDA")


def _group_members(x, rot_idx, rot_cs, scales, krot, wpack, wmeta, bias, out_dtype):
    """The pq_linear_member table of a group over x [.., k], the outputs it writes, and what must stay alive."""
    dev = x.device
    count = len(wpack)
    _require(1 <= count <= _lib.MAX_GROUP, f"a group holds 1..{_lib.MAX_GROUP} linears, got {count}")
    _require(len(rot_idx) == len(rot_cs) == len(scales) == len(wmeta) == len(bias) == count,
             "every per-member list must have one entry per linear")
    _require(out_dtype in _DT, f"out_dtype must be float32/float16/bfloat16, got {out_dtype}")
    k = x.size(-1)
    m = x.numel() // k
    members = (_lib.LinearMember * count)()
    keep, outs, bias_dt = [], [], 0
    for i in range(count):
        n, kw = _check_weights(wpack[i], wmeta[i], dev)
        _require(kw == k, f"member {i}: the weights expect {kw} features, x has {k}")
        _check_rot_params(x, rot_idx[i], rot_cs[i], scales[i], krot)
        idx, cs = rot_idx[i].contiguous(), rot_cs[i].contiguous()
        sc = scales[i].contiguous() if scales[i] is not None else None
        b = bias[i]
        if b is not None:
            _require(b.dtype in _DT and b.numel() == n, f"member {i}: bias must hold {n} float values")
            _same_device("bias", b, dev)
            b = b.contiguous()
            _require(bias_dt in (0, _DT[b.dtype]), "all biases of a group must share one dtype")
            bias_dt = _DT[b.dtype]
        y = torch.empty((m, n), dtype=out_dtype, device=dev)
        keep += [idx, cs, sc, b]
        outs.append(y)
        members[i] = _lib.LinearMember(idx.data_ptr(), cs.data_ptr(), sc.data_ptr() if sc is not None else None,
                                       wpack[i].data_ptr(), wmeta[i].data_ptr(),
                                       b.data_ptr() if b is not None else None, y.data_ptr(), n)
    return members, outs, keep, bias_dt, m, k


def _group_scratch(m, k, count, dev):
    """Scratch of a group launch from torch's caching allocator (inside a graph capture: the graph's pool,
    at fixed addresses across replays)."""
    need = int(_lib.load().pq_w4a8_linear_group_workspace_size(m, k, count))
    return torch.empty(need, dtype=torch.uint8, device=dev) if need > 0 else None


def _linear_group_impl(x, rot_idx, rot_cs, scales, krot, wpack, wmeta, bias, input_fp16, materialize_fp16,
                       out_dtype):
    dev = x.device
    xc = x.contiguous()
    members, outs, keep, bias_dt, m, k = _group_members(xc, rot_idx, rot_cs, scales, krot, wpack, wmeta, bias,
                                                        out_dtype)
    count = len(outs)
    scratch = _group_scratch(m, k, count, dev)
    flags = (_lib.PQ_RQ_INPUT_FP16 if input_fp16 else 0) | (_lib.PQ_RQ_MATERIALIZE_FP16 if materialize_fp16 else 0)
    lib = _lib.load()
    with _DeviceGuard(dev):
        st = lib.pq_w4a8_linear_group(xc.data_ptr(), _DT[x.dtype], members, count, bias_dt, _DT[out_dtype], m, k,
                                      krot, flags, scratch.data_ptr() if scratch is not None else None,
                                      scratch.numel() if scratch is not None else 0, _stream(dev))
    _lib.check(st, "paroquant::w4a8_linear_group")
    return [y.view(*x.shape[:-1], y.size(1)) for y in outs]


def _linear_group_fused_impl(x, x2, norm_weight, eps, mode, rot_idx, rot_cs, scales, krot, wpack, wmeta, bias,
                             input_fp16, materialize_fp16, out_dtype, return_h, return_sum):
    dev = x.device
    _require(x.dtype in _DT, f"x must be float32/float16/bfloat16, got {x.dtype}")
    _require(mode in (_lib.PQ_PRO_RMSNORM, _lib.PQ_PRO_ADD, _lib.PQ_PRO_SWIGLU), f"unknown prologue mode {mode}")
    xc = x.contiguous()
    k = xc.size(-1)
    w = None
    if mode == _lib.PQ_PRO_RMSNORM:
        _require(norm_weight is not None and norm_weight.dtype == x.dtype and norm_weight.numel() == k,
                 f"norm_weight must hold {k} values of x's dtype {x.dtype}")
        _same_device("norm_weight", norm_weight, dev)
        w = norm_weight.contiguous()
    else:
        _require(x2 is not None, "the add and the SwiGLU need x2 (residual / up)")
    other = None
    if x2 is not None:
        _require(x2.shape == x.shape and x2.dtype == x.dtype, "x2 (residual / up) must match x's shape and dtype")
        _same_device("x2", x2, dev)
        other = x2.contiguous()
    _require(not return_sum or (other is not None and mode != _lib.PQ_PRO_SWIGLU),
             "return_sum needs a residual (RMSNorm with residual, or the add)")
    _require(not return_h or mode != _lib.PQ_PRO_ADD, "the add has no h: use return_sum")
    members, outs, keep, bias_dt, m, _ = _group_members(xc, rot_idx, rot_cs, scales, krot, wpack, wmeta, bias,
                                                        out_dtype)
    count = len(outs)
    h = torch.empty_like(xc) if return_h else None
    sm = torch.empty_like(xc) if return_sum else None
    scratch = _group_scratch(m, k, count, dev)
    flags = (_lib.PQ_RQ_INPUT_FP16 if input_fp16 else 0) | (_lib.PQ_RQ_MATERIALIZE_FP16 if materialize_fp16 else 0)
    lib = _lib.load()
    with _DeviceGuard(dev):
        st = lib.pq_w4a8_linear_group_fused(
            xc.data_ptr(), other.data_ptr() if other is not None else None, w.data_ptr() if w is not None else None,
            float(eps), int(mode), h.data_ptr() if h is not None else None,
            sm.data_ptr() if sm is not None else None, _DT[x.dtype], members, count, bias_dt, _DT[out_dtype], m, k,
            krot, flags, scratch.data_ptr() if scratch is not None else None,
            scratch.numel() if scratch is not None else 0, _stream(dev))
    _lib.check(st, "paroquant::w4a8_linear_group_fused")
    res_out = [y.view(*x.shape[:-1], y.size(1)) for y in outs]
    if h is not None:
        res_out.append(h.view(x.shape))
    if sm is not None:
        res_out.append(sm.view(x.shape))
    return res_out


_pq_lib.impl("w4a8_linear_group_fused", _linear_group_fused_impl, "CUDA")


@torch.library.register_fake("paroquant::w4a8_linear_group_fused")
def _linear_group_fused_fake(x, x2, norm_weight, eps, mode, rot_idx, rot_cs, scales, krot, wpack, wmeta, bias,
                             input_fp16, materialize_fp16, out_dtype, return_h, return_sum):
    outs = [x.new_empty((*x.shape[:-1], w.size(0) * 16), dtype=out_dtype) for w in wpack]
    if return_h:
        outs.append(x.new_empty(x.shape))
    if return_sum:
        outs.append(x.new_empty(x.shape))
    return outs


def _linear_group_rmsnorm_impl(x, residual, norm_weight, eps, rot_idx, rot_cs, scales, krot, wpack, wmeta, bias,
                               input_fp16, materialize_fp16, out_dtype, return_normed, return_sum):
    return _linear_group_fused_impl(x, residual, norm_weight, eps, _lib.PQ_PRO_RMSNORM, rot_idx, rot_cs, scales, krot,
                                    wpack, wmeta, bias, input_fp16, materialize_fp16, out_dtype, return_normed,
                                    return_sum)


_pq_lib.impl("w4a8_linear_group_rmsnorm", _linear_group_rmsnorm_impl, "CUDA")


@torch.library.register_fake("paroquant::w4a8_linear_group_rmsnorm")
def _linear_group_rmsnorm_fake(x, residual, norm_weight, eps, rot_idx, rot_cs, scales, krot, wpack, wmeta, bias,
                               input_fp16, materialize_fp16, out_dtype, return_normed, return_sum):
    outs = [x.new_empty((*x.shape[:-1], w.size(0) * 16), dtype=out_dtype) for w in wpack]
    if return_normed:
        outs.append(x.new_empty(x.shape))
    if return_sum:
        outs.append(x.new_empty(x.shape))
    return outs


_pq_lib.impl("w4a8_linear_group", _linear_group_impl, "CUDA")


@torch.library.register_fake("paroquant::w4a8_linear_group")
def _linear_group_fake(x, rot_idx, rot_cs, scales, krot, wpack, wmeta, bias, input_fp16, materialize_fp16,
                       out_dtype):
    return [x.new_empty((*x.shape[:-1], w.size(0) * 16), dtype=out_dtype) for w in wpack]


def split_path(m, k) -> bool:
    """True when the linear entry points run m tokens of k features on the split-rotation kernels: the rule of
    pq_w4a8_linear_split_path, restated in Python so that torch.compile can guard on it when m is a symbolic
    size (tests check the two agree).  Split pair: m * k <= 8192, or k >= 8192 and m <= 2, as long as the
    GEMM's LDS image of A fits (m <= 16, m * (k + 16) <= 80 KiB); three-launch rows: otherwise
    k in [4096, 16384] and m <= 64."""
    if m < 1 or k % 128 or k > 16384:
        return False
    split = (m * k <= 8192 or (k >= 8192 and m <= 2)) and m <= 16 and m * (k + 16) <= 80 * 1024
    return bool(split or (m <= 64 and k >= 4096))


def linear_group_workspace_bytes(m: int, k: int, count: int) -> int:
    """Workspace bytes paroquant::w4a8_linear_group needs for count linears over an [m, k] input."""
    return int(_lib.load().pq_w4a8_linear_group_workspace_size(m, k, count))


class W4A8GroupStages:
    """paroquant::w4a8_linear_group (or _fused with a prologue) split into its two stages
    (pq_w4a8_linear_group_stage): ``rotate()`` makes the rotation (+ quant) launches into a workspace this
    object owns, ``gemm()`` the GEMM launch from it, writing ``outs``.  Both enqueue on the current stream and
    may be captured in graphs, separately.  Built once for fixed inputs and outputs (their addresses are
    baked into the calls)."""

    def __init__(self, x, rot_idx, rot_cs, scales, krot, wpack, wmeta, bias, input_fp16=True,
                 materialize_fp16=True, out_dtype=torch.bfloat16, x2=None, norm_weight=None, eps=0.0, mode=0):
        self.dev = x.device
        self.x = x.contiguous()
        self.x2 = x2.contiguous() if x2 is not None else None
        self.w = norm_weight.contiguous() if norm_weight is not None else None
        self.members, self.outs, self._keep, self.bias_dt, self.m, self.k = _group_members(
            self.x, rot_idx, rot_cs, scales, krot, wpack, wmeta, bias, out_dtype)
        self.count = len(self.outs)
        self.krot, self.eps, self.mode, self.out_dt = krot, float(eps), int(mode), _DT[out_dtype]
        self.flags = ((_lib.PQ_RQ_INPUT_FP16 if input_fp16 else 0)
                      | (_lib.PQ_RQ_MATERIALIZE_FP16 if materialize_fp16 else 0))
        self.scratch = _group_scratch(self.m, self.k, self.count, self.dev)

    def _call(self, stage):
        lib = _lib.load()
        sc = self.scratch
        with _DeviceGuard(self.dev):
            st = lib.pq_w4a8_linear_group_stage(
                stage, self.x.data_ptr(), self.x2.data_ptr() if self.x2 is not None else None,
                self.w.data_ptr() if self.w is not None else None, self.eps, self.mode, None, None, _DT[self.x.dtype],
                self.members, self.count, self.bias_dt, self.out_dt, self.m, self.k, self.krot, self.flags,
                sc.data_ptr() if sc is not None else None, sc.numel() if sc is not None else 0, _stream(self.dev))
        _lib.check(st, f"pq_w4a8_linear_group_stage({stage})")

    def rotate(self):
        self._call(1)

    def gemm(self):
        self._call(2)
        return self.outs


def w4a8_linear_group_intermediates(x, rot_idx, rot_cs, scales, krot, wpack, wmeta, input_fp16=True,
                                    materialize_fp16=True, x2=None, norm_weight=None, eps=0.0, mode=0,
                                    return_h=False, return_sum=False):
    """Parity probe of the grouped W4A8 linear (pq_w4a8_linear_group_intermediates; not a torch op and not a
    fast path).  Runs the launches paroquant::w4a8_linear_group (mode 0) or
    paroquant::w4a8_linear_group_fused (mode PQ_PRO_*, with x2 / norm_weight / eps as there) make for these
    sizes, with the GEMM in its partials form, and returns per member what that GEMM multiplied and summed:
    (codes int8 [count, m, k], xscale float32 [count, m], [partials int32 [m, k/128, n_i] per member],
    h or None, s or None)."""
    dev = x.device
    _require(x.dtype in _DT, f"x must be float32/float16/bfloat16, got {x.dtype}")
    xc = x.contiguous()
    k = xc.size(-1)
    nb = [None] * len(wpack)
    members, _, keep, _, m, _ = _group_members(xc, rot_idx, rot_cs, scales, krot, wpack, wmeta, nb, torch.bfloat16)
    count = len(wpack)
    G = k // 128
    codes = torch.empty((count, m, k), dtype=torch.int8, device=dev)
    xscale = torch.empty((count, m), dtype=torch.float32, device=dev)
    ns = [int(members[i].n) for i in range(count)]
    flat = torch.empty(m * G * sum(ns), dtype=torch.int32, device=dev)
    parts, off = [], 0
    for n in ns:
        parts.append(flat[off:off + m * G * n].view(m, G, n))
        off += m * G * n
    other = x2.contiguous() if x2 is not None else None
    w = norm_weight.contiguous() if norm_weight is not None else None
    h = torch.empty_like(xc) if return_h else None
    sm = torch.empty_like(xc) if return_sum else None
    scratch = _group_scratch(m, k, count, dev)
    flags = (_lib.PQ_RQ_INPUT_FP16 if input_fp16 else 0) | (_lib.PQ_RQ_MATERIALIZE_FP16 if materialize_fp16 else 0)
    lib = _lib.load()
    with _DeviceGuard(dev):
        st = lib.pq_w4a8_linear_group_intermediates(
            xc.data_ptr(), other.data_ptr() if other is not None else None, w.data_ptr() if w is not None else None,
            float(eps), int(mode), h.data_ptr() if h is not None else None,
            sm.data_ptr() if sm is not None else None, _DT[x.dtype], members, count, m, k, krot, flags,
            scratch.data_ptr() if scratch is not None else None, scratch.numel() if scratch is not None else 0,
            codes.data_ptr(), xscale.data_ptr(), flat.data_ptr(), _stream(dev))
    _lib.check(st, "pq_w4a8_linear_group_intermediates")
    del keep
    return codes, xscale, parts, h, sm


@torch.library.register_fake("paroquant::w4a8_linear")
def _linear_fake(x, rot_idx, rot_cs, scales, krot, wpack, wmeta, bias, input_fp16, materialize_fp16, out_dtype):
    return x.new_empty((*x.shape[:-1], wpack.size(0) * 16), dtype=out_dtype)


# ---------------------------------------------------------------------------
# paroquant::w4a16_prepack / w4a16_gemm / w4a16_linear (WQLinear's W4A16 path)
# ---------------------------------------------------------------------------

def _w16_bias(bias, n, dev):
    if bias is None:
        return None
    _require(bias.dtype in _DT and bias.numel() == n, f"bias must hold {n} float values")
    _same_device("bias", bias, dev)
    return bias.contiguous()


def _w16_prepack_impl(awq_qweight, scales, scaled_zeros):
    dev = awq_qweight.device
    _require(awq_qweight.dtype == torch.int32 and awq_qweight.dim() == 2, "awq_qweight must be int32 [K, N/8]")
    k, n = awq_qweight.size(0), awq_qweight.size(1) * 8
    _require(k % 128 == 0 and n % 16 == 0, f"K={k} must be a multiple of 128 and N={n} of 16")
    g = k // 128
    for name, t in (("scales", scales), ("scaled_zeros", scaled_zeros)):
        _require(t.dtype == torch.float16 and tuple(t.shape) == (g, n),
                 f"{name} must be float16 [{g}, {n}], got {t.dtype} {tuple(t.shape)}")
        _same_device(name, t, dev)
    qw, sc, sz = awq_qweight.contiguous(), scales.contiguous(), scaled_zeros.contiguous()
    wpack = torch.empty((n // 16, g, 64, 16), dtype=torch.uint8, device=dev)
    wmeta = torch.empty((n // 16, g, 16), dtype=torch.int32, device=dev)
    lib = _lib.load()
    with _DeviceGuard(dev):
        st = lib.pq_w4a16_prepack(qw.data_ptr(), sc.data_ptr(), sz.data_ptr(), wpack.data_ptr(), wmeta.data_ptr(), k,
                                  n, 128, _stream(dev))
    _lib.check(st, "paroquant::w4a16_prepack")
    return wpack, wmeta


_pq_lib.impl("w4a16_prepack", _w16_prepack_impl, "CUDA")


@torch.library.register_fake("paroquant::w4a16_prepack")
def _w16_prepack_fake(awq_qweight, scales, scaled_zeros):
    k, n = awq_qweight.size(0), awq_qweight.size(1) * 8
    return (awq_qweight.new_empty((n // 16, k // 128, 64, 16), dtype=torch.uint8),
            awq_qweight.new_empty((n // 16, k // 128, 16), dtype=torch.int32))


def _w16_gemm_impl(x, wpack, wmeta, bias, out_dtype):
    dev = x.device
    n, k = _check_weights(wpack, wmeta, dev)
    _require(x.dtype == torch.float16, f"x must be float16 (the W4A16 kernels take fp16 activations), got {x.dtype}")
    _require(x.size(-1) == k, f"x has {x.size(-1)} features, the weights expect {k}")
    _require(out_dtype in _DT, f"out_dtype must be float32/float16/bfloat16, got {out_dtype}")
    xc = x.contiguous()
    m = xc.numel() // k
    y = torch.empty((m, n), dtype=out_dtype, device=dev)
    bias = _w16_bias(bias, n, dev)
    lib = _lib.load()
    with _DeviceGuard(dev):
        st = lib.pq_w4a16_gemm(xc.data_ptr(), wpack.data_ptr(), wmeta.data_ptr(),
                               bias.data_ptr() if bias is not None else None,
                               _DT[bias.dtype] if bias is not None else 0, y.data_ptr(), _DT[out_dtype], m, n, k, 128,
                               _stream(dev))
    _lib.check(st, "paroquant::w4a16_gemm")
    return y.view(*x.shape[:-1], n)


_pq_lib.impl("w4a16_gemm", _w16_gemm_impl, "CUDA")


@torch.library.register_fake("paroquant::w4a16_gemm")
def _w16_gemm_fake(x, wpack, wmeta, bias, out_dtype):
    return x.new_empty((*x.shape[:-1], wpack.size(0) * 16), dtype=out_dtype)


def w4a16_linear_workspace_bytes(m: int, k: int) -> int:
    return int(_lib.load().pq_w4a16_linear_workspace_size(m, k))


def _w16_linear_impl(x, rot_idx, rot_cs, scales, krot, wpack, wmeta, bias, input_fp16, out_dtype):
    dev = x.device
    n, k = _check_weights(wpack, wmeta, dev)
    _require(x.size(-1) == k, f"x has {x.size(-1)} features, the weights expect {k}")
    _check_rot_params(x, rot_idx, rot_cs, scales, krot)
    _require(out_dtype in _DT, f"out_dtype must be float32/float16/bfloat16, got {out_dtype}")
    xc = x.contiguous()
    m = xc.numel() // k
    y = torch.empty((m, n), dtype=out_dtype, device=dev)
    bias = _w16_bias(bias, n, dev)
    lib = _lib.load()
    need = int(lib.pq_w4a16_linear_workspace_size(m, k))
    scratch = torch.empty(need, dtype=torch.uint8, device=dev) if need > 0 else None
    flags = _lib.PQ_RQ_INPUT_FP16 if input_fp16 else 0
    idx, cs = rot_idx.contiguous(), rot_cs.contiguous()
    sc = scales.contiguous() if scales is not None else None
    with _DeviceGuard(dev):
        st = lib.pq_w4a16_linear(xc.data_ptr(), _DT[x.dtype], idx.data_ptr(), cs.data_ptr(),
                                 sc.data_ptr() if sc is not None else None, wpack.data_ptr(), wmeta.data_ptr(),
                                 bias.data_ptr() if bias is not None else None,
                                 _DT[bias.dtype] if bias is not None else 0, y.data_ptr(), _DT[out_dtype], m, n, k,
                                 krot, flags, scratch.data_ptr() if scratch is not None else None,
                                 scratch.numel() if scratch is not None else 0, _stream(dev))
    _lib.check(st, "paroquant::w4a16_linear")
    return y.view(*x.shape[:-1], n)


_pq_lib.impl("w4a16_linear", _w16_linear_impl, "CUDA")


def _w16_linear_group_impl(x, rot_idx, rot_cs, scales, krot, wpack, wmeta, bias, input_fp16, out_dtype):
    """paroquant::w4a16_linear for linears that read the same x, in one rotation launch and (m <= 16) one GEMM."""
    dev = x.device
    _require(x.dtype in _DT, f"x must be float32/float16/bfloat16, got {x.dtype}")
    xc = x.contiguous()
    members, outs, keep, bias_dt, m, k = _group_members(xc, rot_idx, rot_cs, scales, krot, wpack, wmeta, bias,
                                                        out_dtype)
    count = len(outs)
    lib = _lib.load()
    need = int(lib.pq_w4a16_linear_group_workspace_size(m, k, count))
    scratch = torch.empty(need, dtype=torch.uint8, device=dev) if need > 0 else None
    flags = _lib.PQ_RQ_INPUT_FP16 if input_fp16 else 0
    with _DeviceGuard(dev):
        st = lib.pq_w4a16_linear_group(xc.data_ptr(), _DT[x.dtype], members, count, bias_dt, _DT[out_dtype], m, k,
                                       krot, flags, scratch.data_ptr() if scratch is not None else None,
                                       scratch.numel() if scratch is not None else 0, _stream(dev))
    _lib.check(st, "paroquant::w4a16_linear_group")
    return [y.view(*x.shape[:-1], y.size(1)) for y in outs]


_pq_lib.impl("w4a16_linear_group", _w16_linear_group_impl, "CUDA")


@torch.library.register_fake("paroquant::w4a16_linear_group")
def _w16_linear_group_fake(x, rot_idx, rot_cs, scales, krot, wpack, wmeta, bias, input_fp16, out_dtype):
    return [x.new_empty((*x.shape[:-1], w.size(0) * 16), dtype=out_dtype) for w in wpack]


@torch.library.register_fake("paroquant::w4a16_linear")
def _w16_linear_fake(x, rot_idx, rot_cs, scales, krot, wpack, wmeta, bias, input_fp16, out_dtype):
    return x.new_empty((*x.shape[:-1], wpack.size(0) * 16), dtype=out_dtype)
