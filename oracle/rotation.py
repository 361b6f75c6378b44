"""Oracle: pairwise Givens rotation with channel scales (numpy, CPU).

Restates kernels/paroquant_kernels/src/rotation.cuh:247-337 (``RotateAccess``
load_group / load_coeffs / apply_one / store_group) and the launcher shape
logic of rotation.cu:116-137:

  * x is viewed as [rows, h] with rows = numel / h (rotation.cu:127-128);
  * per 128- (or 64-) channel group, values are loaded to fp32 and
    multiplied by the channel scale (rotation.cuh:261-277);
  * layer r, pair t of group g uses the group-local indices
    i = idx[r, g*G + 2t], j = idx[r, g*G + 2t + 1] (rotation.cuh:291-295)
    and angle theta[r, g*G/2 + t];
  * xi' = c*xi + s*xj,  xj' = -s*xi + c*xj  (rotation.cuh:310-313);
  * the result is rounded to the output dtype (rotation.cuh:333-334).

The floating-point sequence is spelled out so the HIP kernels can reproduce
it bit for bit: cos/sin are evaluated in float64 from the float32 value of
theta and rounded to float32, and each update is
``xi' = fma(xi, c, xj*s)``, ``xj' = fma(xj, c, -(xi*s))`` in float32.
"""

from __future__ import annotations

import numpy as np


def cos_sin_table(theta: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """float32 (cos, sin) of theta, evaluated in float64 then rounded."""
    t = np.asarray(theta).astype(np.float32).astype(np.float64)
    return np.cos(t).astype(np.float32), np.sin(t).astype(np.float32)


def _fma32(a: np.ndarray, b: np.ndarray, c: np.ndarray) -> np.ndarray:
    # a*b is exact in float64 (24+24 bits), so this is fma up to a double
    # rounding that only matters within 2^-29 of an fp32 midpoint.
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(np.float32)


def pair_index_arrays(pairs: np.ndarray, group_size: int) -> tuple[np.ndarray, np.ndarray]:
    """Absolute channel indices (i, j) of every pair, shape [krot, h/2].

    Pair t of group g sits at position g*G/2 + t, matching theta's layout.
    """
    pairs = np.asarray(pairs).astype(np.int64)
    krot, h = pairs.shape
    ng = h // group_size
    p = pairs.reshape(krot, ng, group_size)
    base = (np.arange(ng, dtype=np.int64) * group_size)[None, :, None]
    gi = (p[:, :, 0::2] + base).reshape(krot, h // 2)
    gj = (p[:, :, 1::2] + base).reshape(krot, h // 2)
    return gi, gj


def check_pairs(pairs: np.ndarray, group_size: int) -> None:
    """Raise ValueError unless every layer pairs each group's channels disjointly.

    The reference kernel updates all pairs of a layer concurrently in shared
    memory (rotation.cu:47-54), so overlapping pairs are a data race there;
    the oracle requires a perfect matching per group and layer.
    """
    pairs = np.asarray(pairs).astype(np.int64)
    krot, h = pairs.shape
    if h % group_size:
        raise ValueError(f"h={h} is not a multiple of group_size={group_size}")
    if pairs.min(initial=0) < 0 or pairs.max(initial=0) >= group_size:
        raise ValueError("pair indices must be group-local in [0, group_size)")
    p = np.sort(pairs.reshape(krot, h // group_size, group_size), axis=-1)
    if not np.array_equal(p, np.broadcast_to(np.arange(group_size), p.shape)):
        raise ValueError("each layer must pair every channel of a group exactly once")


def rotate_f32(xs: np.ndarray, pairs: np.ndarray, cos: np.ndarray, sin: np.ndarray,
               group_size: int) -> np.ndarray:
    """Apply the Givens layers to already-scaled float32 rows xs [rows, h]."""
    y = np.array(xs, dtype=np.float32, copy=True)
    gi, gj = pair_index_arrays(pairs, group_size)
    for r in range(gi.shape[0]):
        c = cos[r].astype(np.float32)
        s = sin[r].astype(np.float32)
        xi = y[:, gi[r]]
        xj = y[:, gj[r]]
        ni = _fma32(xi, c, (xj * s).astype(np.float32))
        nj = _fma32(xj, c, -(xi * s).astype(np.float32))
        y[:, gi[r]] = ni
        y[:, gj[r]] = nj
    return y


def scale_rows(x: np.ndarray, scales: np.ndarray | None) -> np.ndarray:
    """fp32 load and channel-scale multiply (rotation.cuh:261-277)."""
    xf = np.asarray(x).astype(np.float32)
    if scales is None:
        return xf
    s = np.asarray(scales).astype(np.float32).reshape(-1)
    return (xf * s[None, :]).astype(np.float32)


def rotate(x: np.ndarray, idx_ij: np.ndarray, theta: np.ndarray, scales: np.ndarray | None,
           group_size: int, out_dtype=None) -> np.ndarray:
    """The ``rotation::rotate`` op (rotation.cu:456-493): any leading dims.

    Returns an array of ``out_dtype`` (default: x's dtype) with x's shape.
    """
    x = np.asarray(x)
    h = x.shape[-1]
    if h % group_size:
        raise ValueError("h must be divisible by group_size")
    if theta.shape[0] != idx_ij.shape[0]:
        raise ValueError("theta.size(0) must equal idx_ij.size(0)")
    rows = x.reshape(-1, h)
    c, s = cos_sin_table(theta)
    y = rotate_f32(scale_rows(rows, scales), idx_ij, c, s, group_size)
    dt = x.dtype if out_dtype is None else out_dtype
    return y.astype(dt).reshape(x.shape)


def rotate_path_f32(x_bf16_as_f32: np.ndarray, pairs: np.ndarray, cos: np.ndarray,
                    sin: np.ndarray, scales_f32: np.ndarray | None, group_size: int = 128,
                    input_fp16: bool = True, materialize_fp16: bool = True) -> np.ndarray:
    """Rotation as the W4A8 linear sees it (paroquant_marlin_w4a8.py:59-65).

    The wrapper casts the bf16 activations to fp16 before the rotation
    (``input_fp16``) and the fp16 kernel stores its result rounded to fp16
    (``materialize_fp16``) before vLLM quantizes it.  Returns float32.
    """
    xf = np.asarray(x_bf16_as_f32, dtype=np.float32)
    if input_fp16:
        xf = xf.astype(np.float16).astype(np.float32)
    y = rotate_f32(scale_rows(xf, scales_f32), pairs, cos, sin, group_size)
    if materialize_fp16:
        y = y.astype(np.float16).astype(np.float32)
    return y


def unpack_packed_params(rot_idx: np.ndarray, rot_cs: np.ndarray, krot: int):
    """Packed kernel operands -> (init, Af, Bf, src, flag, cos, sin).

    rot_idx [G, 64, KP/2] uint32: word 0 = Af | Bf << 8 | init << 16 (channels
    in slots A/B after the last layer; slot A starts with channel lane+64 when
    init is set, else with channel lane); byte 4 + r = src | flag << 7 for the
    fetch before layer r.  rot_cs [G, 64, KP, 2] float32.
    src / flag / cos / sin are [G, 64, krot].
    """
    w = np.ascontiguousarray(rot_idx).view(np.uint32)
    b = w.view(np.uint8).reshape(w.shape[0], w.shape[1], -1).astype(np.int64)
    w0 = w[:, :, 0].astype(np.int64)
    Af, Bf = w0 & 0xFF, (w0 >> 8) & 0xFF
    init = ((w0 >> 16) & 1) != 0
    src = b[:, :, 4:4 + krot] & 0x3F
    flag = (b[:, :, 4:4 + krot] >> 7) != 0
    cs = np.asarray(rot_cs, np.float32)[:, :, :krot]
    return init, Af, Bf, src, flag, cs[..., 0], cs[..., 1]


def rotate_f32_packed(xs: np.ndarray, rot_idx: np.ndarray, rot_cs: np.ndarray, krot: int) -> np.ndarray:
    """The kernels' use of the packed operands, lane by lane: lane l loads
    channels l and l+64 into slots (a, b) (swapped when init is set); before
    layer r it fetches slot a of lane src and puts it into slot a (flag) or b,
    keeping its old slot b in the other; every layer is a' = fma(a, c, b*s),
    b' = fma(b, c, -(a*s)); at the end slot a holds channel Af and b channel Bf."""
    x = np.asarray(xs, dtype=np.float32)
    init, Af, Bf, src, flag, c, s = unpack_packed_params(rot_idx, rot_cs, krot)
    G = init.shape[0]
    rows = x.shape[0]
    xg = x.reshape(rows, G, 128)
    gi = np.arange(G)[:, None]
    lo, hi = xg[:, :, :64], xg[:, :, 64:]
    a = np.where(init[None], hi, lo)          # [rows, G, 64]
    b = np.where(init[None], lo, hi)
    for r in range(krot):
        recv = a[:, gi, src[:, :, r]]
        fl = flag[:, :, r][None]
        a, b = np.where(fl, recv, b), np.where(fl, b, recv)
        cr = c[:, :, r][None]
        sr = s[:, :, r][None]
        na = _fma32(a, cr, (b * sr).astype(np.float32))
        nb = _fma32(b, cr, -(a * sr).astype(np.float32))
        a, b = na, nb
    y = np.empty_like(xg)
    y[:, gi, Af] = a
    y[:, gi, Bf] = b
    return y.reshape(rows, G * 128)


def rotate_backward(x: np.ndarray, pairs: np.ndarray, theta: np.ndarray, scales: np.ndarray | None,
                    grad_y: np.ndarray, group_size: int):
    """Gradients of y = R_{K-1} ... R_0 (s * x) with respect to x, theta and s, in float64.

    Layer r maps a pair (a, b) to (a', b') = (c a + s b, c b - s a), so
    d(a', b')/d theta = (b', -a'): the angle's gradient is
    sum_rows (g_a' b' - g_b' a'), with (g_a', g_b') the gradient at the layer's
    output, and the gradient at its input is the transposed rotation
    (c g_a' - s g_b', s g_a' + c g_b').  The layers' outputs are recomputed
    forward from x (not recovered by inverting y).  Below layer 0 the gradient
    g_t is taken at t = s * x: d x = s * g_t and d s = sum_rows x * g_t.
    cos / sin are those of cos_sin_table (the float32 values the kernels use).
    Returns (grad_x [rows, h], grad_theta [krot, h/2], grad_scales [h] or None).
    The values are those of the reference's RotateTensorFunc.backward
    (kernels/paroquant_kernels/interface.py:30-93), which reaches them another way.
    """
    x = np.asarray(x, np.float64)
    h = x.shape[-1]
    xr = x.reshape(-1, h)
    c32, s32 = cos_sin_table(theta)
    c, s = c32.astype(np.float64), s32.astype(np.float64)
    gi, gj = pair_index_arrays(pairs, group_size)
    krot = gi.shape[0]
    sc = None if scales is None else np.asarray(scales, np.float64).reshape(-1)
    t = xr * sc[None, :] if sc is not None else xr.copy()
    outs = []
    for r in range(krot):
        a, b = t[:, gi[r]], t[:, gj[r]]
        na, nb = c[r] * a + s[r] * b, c[r] * b - s[r] * a
        t[:, gi[r]], t[:, gj[r]] = na, nb
        outs.append((na, nb))
    g = np.asarray(grad_y, np.float64).reshape(-1, h).copy()
    g_theta = np.zeros((krot, h // 2))
    for r in range(krot - 1, -1, -1):
        na, nb = outs[r]
        ga, gb = g[:, gi[r]], g[:, gj[r]]
        g_theta[r] = (ga * nb - gb * na).sum(axis=0)
        g[:, gi[r]], g[:, gj[r]] = c[r] * ga - s[r] * gb, s[r] * ga + c[r] * gb
    if sc is None:
        return g, g_theta, None
    return g * sc[None, :], g_theta, (xr * g).sum(axis=0)
