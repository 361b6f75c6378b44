"""Oracle: int4 weight layouts (numpy, CPU).

Three layouts meet on the W4A8 path:

  * WQLinear int16 [N/4, K] -- ParoQuant checkpoints
    (src/alpamayo_r1/utils/quantization/qmodule.py:39-78 ``pack_intweight``,
    inverse paroquant_marlin_w4a8.py:95-142 ``unpack_wqlinear_qweight``);
  * AWQ int32 [K, N/8] with nibble order [0, 2, 4, 6, 1, 3, 5, 7]
    (paroquant_marlin_w4a8.py:149-164 ``pack_awq_int32``), which is what
    ``MarlinW4A8Linear.load_from_awq`` consumes (paroquant_marlin_w4a8.py:274);
  * this project's kernel layout ``wpack``/``wmeta`` (defined here; it is the
    specification the HIP prepack kernel must reproduce bit for bit).

The permutations are written as explicit index maps rather than as the
reference's reshape/transpose chains; tests pin them against golden vectors
produced by the reference's own ``pack_intweight``.
"""

from __future__ import annotations

import numpy as np

AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)   # paroquant_marlin_w4a8.py:149


# --------------------------------------------------------------------------
# WQLinear (qmodule.py:24-78)
# --------------------------------------------------------------------------

def make_divisible(c: int, divisor: int) -> int:
    return (c + divisor - 1) // divisor


def calculate_zeros_width(in_features: int, group_size: int = 128, pack_num: int = 8) -> int:
    """Row count (/8) of WQLinear's scales/scaled_zeros buffers (qmodule.py:24-36)."""
    if group_size >= 128:
        mult = 1
    elif group_size == 64:
        mult = 2
    elif group_size == 32:
        mult = 4
    else:
        raise NotImplementedError(group_size)
    base = make_divisible(in_features // group_size, pack_num)
    return make_divisible(base, mult) * mult


def _wq_k_source(K: int) -> np.ndarray:
    """For each packed K position, the original K index it holds.

    Inside each block of 32, position p = 8a + 4c + b holds original index
    8b + 2a + c (two K shuffles of qmodule.py:45-55 composed).
    """
    p = np.arange(32)
    a, rem = p // 8, p % 8
    c, b = rem // 4, rem % 4
    src32 = 8 * b + 2 * a + c
    blocks = np.arange(K // 32)[:, None] * 32
    return (blocks + src32[None, :]).reshape(K)


def pack_intweight(unpacked: np.ndarray, interleave: int = 4, kstride: int = 64) -> np.ndarray:
    """int4 codes [N, K] -> WQLinear int16 [N/interleave, K] (qmodule.py:39-78)."""
    w = np.asarray(unpacked).astype(np.int64)
    N, K = w.shape
    shuffled = w[:, _wq_k_source(K)]                     # K shuffles
    # Row interleave: a 4 x 64 tile (rows 4*nb..4*nb+3, cols kb*64..) is
    # re-read as 64 x 4; element (e, f) of the new view is flat index 4e+f.
    nb = N // interleave
    tiles = shuffled.reshape(nb, interleave, K // kstride, kstride).transpose(0, 2, 1, 3)
    tiles = tiles.reshape(nb, K // kstride, kstride, interleave)   # flat reinterpretation
    packed = np.zeros((nb, K // kstride, kstride), dtype=np.int64)
    for f in range(interleave):
        packed |= (tiles[..., f] & 0xF) << (4 * f)
    return packed.reshape(nb, K).astype(np.uint16).view(np.int16)


def unpack_wqlinear_qweight(qweight: np.ndarray, out_features: int, in_features: int,
                            interleave: int = 4, kstride: int = 64) -> np.ndarray:
    """WQLinear int16 [N/4, K] -> int4 codes [N, K] int32 (paroquant_marlin_w4a8.py:95-142)."""
    N, K = out_features, in_features
    pw = np.asarray(qweight).view(np.uint16).astype(np.int64).reshape(N // interleave, K // kstride, kstride)
    nib = np.stack([(pw >> (4 * f)) & 0xF for f in range(interleave)], axis=-1)
    tiles = nib.reshape(N // interleave, K // kstride, interleave, kstride).transpose(0, 2, 1, 3)
    shuffled = tiles.reshape(N, K)
    out = np.empty_like(shuffled)
    out[:, _wq_k_source(K)] = shuffled
    return out.astype(np.int32)


# --------------------------------------------------------------------------
# AWQ int32 (paroquant_marlin_w4a8.py:149-209)
# --------------------------------------------------------------------------

def pack_awq_int32(values: np.ndarray) -> np.ndarray:
    """[rows, cols] int4 -> [rows, cols/8] int32; nibble i holds column 8c + AWQ_ORDER[i]."""
    v = np.asarray(values).astype(np.int64)
    rows, cols = v.shape
    if cols % 8:
        raise ValueError(f"cols={cols} must be divisible by 8")
    v = v.reshape(rows, cols // 8, 8)
    out = np.zeros((rows, cols // 8), dtype=np.int64)
    for i, src in enumerate(AWQ_ORDER):
        out |= (v[:, :, src] & 0xF) << (4 * i)
    return out.astype(np.uint32).view(np.int32)


def unpack_awq_int32(packed: np.ndarray, cols: int) -> np.ndarray:
    p = np.asarray(packed).view(np.uint32).astype(np.int64)
    rows = p.shape[0]
    out = np.empty((rows, cols // 8, 8), dtype=np.int32)
    for i, dst in enumerate(AWQ_ORDER):
        out[:, :, dst] = (p >> (4 * i)) & 0xF
    return out.reshape(rows, cols)


def wqlinear_to_awq(qweight_i16, scales, scaled_zeros, out_features, in_features, group_size):
    """WQLinear buffers -> (awq_qweight [K, N/8], awq_scales fp16 [G, N], awq_qzeros [G, N/8],
    codes [N, K], zeros [G, N]) (paroquant_marlin_w4a8.py:179-209).

    Zero points come back as round(-scaled_zeros / scales) clamped to [0, 15],
    with near-zero scales treated as 1.
    """
    N, K = out_features, in_features
    G = K // group_size
    codes = unpack_wqlinear_qweight(qweight_i16, N, K)
    awq_qweight = pack_awq_int32(codes.T)
    awq_scales = np.asarray(scales)[:G, :N].astype(np.float16)
    sc = awq_scales.astype(np.float32)
    sc = np.where(np.abs(sc) < 1e-10, np.float32(1.0), sc)
    sz = np.asarray(scaled_zeros)[:G, :N].astype(np.float32)
    zeros = np.clip(np.rint(-sz / sc), 0, 15).astype(np.int32)
    return awq_qweight, awq_scales, pack_awq_int32(zeros), codes, zeros


# --------------------------------------------------------------------------
# Kernel layout (this project's own)
# --------------------------------------------------------------------------
#
# wpack: uint8 [N/16][G][64 slots][16 bytes], G = K/128.
#   slot L = 16*j + c holds column n = 16*tile + c and the 32 codes
#   k = 128*g + 32*j + [0, 32).  Byte b of the slot (dword d = b/4, i = b%4)
#   packs code(kb + i) in its low nibble and code(kb + 4 + i) in its high
#   nibble, kb = 128*g + 32*j + 8*d; so one dword's low nibbles are four
#   consecutive k and its high nibbles the next four.
# wmeta: uint32 [N/16][G][16]: bits 0-15 fp16 scale s[g, n], bits 16-23 the
#   zero point z[g, n].

def prepack_kernel_layout(codes_nk: np.ndarray, scales_gn: np.ndarray, zeros_gn: np.ndarray,
                          group_size: int = 128) -> tuple[np.ndarray, np.ndarray]:
    codes = np.asarray(codes_nk).astype(np.uint8)
    N, K = codes.shape
    if group_size != 128 or K % 128 or N % 16:
        raise ValueError("kernel layout needs group_size=128, K%128==0, N%16==0")
    G = K // 128
    # codes -> [tile, c, g, j, d, half, i]: k = 128g + 32j + 8d + 4*half + i
    c6 = codes.reshape(N // 16, 16, G, 4, 4, 2, 4)
    byte = c6[..., 0, :] | (c6[..., 1, :] << 4)            # [tile, c, g, j, d, i]
    byte = byte.reshape(N // 16, 16, G, 4, 16)             # [tile, c, g, j, b]
    wpack = byte.transpose(0, 2, 3, 1, 4).reshape(N // 16, G, 64, 16)   # slot = 16j + c
    sbits = np.asarray(scales_gn).astype(np.float16).view(np.uint16).astype(np.uint32)
    z = np.asarray(zeros_gn).astype(np.uint32) & 0xFF
    meta = (sbits | (z << 16)).T.reshape(N // 16, 16, G).transpose(0, 2, 1)
    return np.ascontiguousarray(wpack), np.ascontiguousarray(meta.astype(np.uint32))


def unpack_kernel_layout(wpack: np.ndarray, wmeta: np.ndarray):
    """Inverse of prepack_kernel_layout -> (codes [N, K], scales fp16 [G, N], zeros [G, N])."""
    T, G = wpack.shape[:2]
    N, K = 16 * T, 128 * G
    byte = np.asarray(wpack).reshape(T, G, 4, 16, 16).transpose(0, 3, 1, 2, 4)  # [tile, c, g, j, b]
    byte = byte.reshape(T, 16, G, 4, 4, 4)
    codes = np.stack([byte & 0xF, byte >> 4], axis=-2)      # [tile, c, g, j, d, half, i]
    codes = codes.reshape(N, K).astype(np.int32)
    meta = np.asarray(wmeta).transpose(0, 2, 1).reshape(N, G).T
    scales = (meta & 0xFFFF).astype(np.uint16).view(np.float16)
    zeros = ((meta >> 16) & 0xFF).astype(np.int32)
    return codes, scales, zeros
