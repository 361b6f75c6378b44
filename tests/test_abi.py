"""The C-ABI library loads on the CPU, exports every symbol the header declares,
and rejects bad arguments on the host before any launch (no GPU needed)."""

import ctypes
import os
import re

import pytest

from alpamayo_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "paroquant_hip.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(pq_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared()
    assert len(names) >= 9
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures must cover the header exactly"


def test_abi_version():
    assert _lib.load().pq_abi_version() == _lib.ABI_VERSION == 1


def _err(lib):
    return lib.pq_last_error().decode()


def test_rotate_argument_checks():
    lib = _lib.load()
    p = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation first
    assert lib.pq_rotate(p, p, p, p, None, 4, 256, 8, 32, 1, None) == 2
    assert "group_size" in _err(lib)
    assert lib.pq_rotate(p, p, p, p, None, 4, 256, 3, 128, 1, None) == 2
    assert "KROT" in _err(lib)
    assert lib.pq_rotate(p, p, p, p, None, 4, 200, 8, 128, 1, None) == 1
    assert "divisible" in _err(lib)
    assert lib.pq_rotate(p, p, p, p, None, 4, 256, 8, 128, 7, None) == 2
    assert lib.pq_rotate(None, None, None, None, None, 4, 256, 8, 128, 1, None) == 1
    assert lib.pq_rotate(None, None, None, None, None, 0, 256, 8, 128, 1, None) == 0  # empty input: no-op


def test_rotate_quant_and_gemm_argument_checks():
    lib = _lib.load()
    p = ctypes.c_void_p(16)
    assert lib.pq_rotate_quant_i8(p, 2, p, p, None, p, p, None, 4, 200, 8, 3, None) == 1
    assert lib.pq_rotate_quant_i8(p, 2, p, p, None, p, p, None, 4, 256, 0, 3, None) == 2
    assert lib.pq_rotate_quant_i8(p, 2, p, p, None, p, p, None, 4, 256, 8, 8, None) == 1
    assert "flags" in _err(lib)
    assert lib.pq_rotate_quant_i8(ctypes.c_void_p(18), 2, p, p, None, p, p, None, 4, 256, 8, 3, None) == 1
    assert lib.pq_rotate_quant_i8(p, 2, ctypes.c_void_p(24), p, None, p, p, None, 4, 256, 8, 3, None) == 1
    assert "aligned" in _err(lib)
    assert lib.pq_w4a8_gemm(p, p, p, p, None, 0, p, 2, 4, 64, 256, 64, None, 0, None) == 2
    assert lib.pq_w4a8_gemm(p, p, p, p, None, 0, p, 2, 4, 60, 256, 128, None, 0, None) == 1
    assert lib.pq_w4a8_gemm(p, p, p, p, None, 0, p, 2, 4, 64, 200, 128, None, 0, None) == 1
    assert lib.pq_w4a8_gemm(p, p, p, p, None, 0, p, 9, 4, 64, 256, 128, None, 0, None) == 2
    assert lib.pq_w4a8_prepack(p, p, p, p, p, 100, 64, 128, None) == 1
    assert lib.pq_w4a8_gemm_partials(p, p, p, p, 0, 64, 256, 128, None) == 0


def test_linear_argument_checks():
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    args = lambda m, k, krot, flags, ws, wsb: (p, 2, p, p, None, p, p, None, 0, p, 2, m, 4096, k, krot, flags, ws, wsb,
                                              None)   # noqa: E731
    assert lib.pq_w4a8_linear(*args(1, 200, 8, 3, None, 0)) == 1
    assert lib.pq_w4a8_linear(*args(1, 4096, 0, 3, None, 0)) == 2
    assert lib.pq_w4a8_linear(*args(1, 4096, 8, 4, None, 0)) == 1
    assert lib.pq_w4a8_linear(*args(1, 32768, 8, 3, None, 0)) == 1
    assert lib.pq_w4a8_linear(*args(0, 4096, 8, 3, None, 0)) == 0
    need = lib.pq_w4a8_linear_workspace_size(65, 4096, 4096, 8)
    assert need == 65 * 4096 + 65 * 4
    assert lib.pq_w4a8_linear(*args(65, 4096, 8, 3, None, 0)) == 4
    assert "workspace" in _err(lib)
    assert lib.pq_w4a8_linear(*args(65, 4096, 8, 3, p, need - 1)) == 4
    assert lib.pq_w4a8_linear(*args(65, 4096, 8, 3, ctypes.c_void_p(272), need)) == 4   # not 256-aligned


def test_linear_group_argument_checks():
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    mem = (_lib.LinearMember * 5)()
    for i in range(5):
        mem[i] = _lib.LinearMember(256, 256, None, 256, 256, None, 256, 64)
    call = lambda members, count, m=2, k=1024: lib.pq_w4a8_linear_group(  # noqa: E731
        p, 2, members, count, 0, 2, m, k, 8, 3, p, 1 << 20, None)
    assert call(mem, 0) == 1 and "count" in _err(lib)
    assert call(mem, 5) == 1
    assert call(None, 2) == 1 and "member table" in _err(lib)
    mem[1].n = 40
    assert call(mem, 2) == 1 and "member 1" in _err(lib)
    mem[1].n = 64
    assert call(mem, 2, k=1000) == 1
    assert call(mem, 2, m=0) == 0                       # empty input: nothing to do
    mem[0].rot_idx = None
    assert call(mem, 2) == 1 and "member 0: null pointer" in _err(lib)
    mem[0].rot_idx = 256
    assert lib.pq_w4a8_linear_group(p, 2, mem, 2, 0, 2, 2, 1024, 8, 3, p, 16, None) == 4   # workspace too small
    # the workspace of a group: count times one member's
    for m, k in ((1, 4096), (3, 4096), (1, 12288), (4, 4096), (300, 2048)):
        one = lib.pq_w4a8_linear_workspace_size(m, 64, k, 8)
        assert lib.pq_w4a8_linear_group_workspace_size(m, k, 3) == 3 * one
    assert lib.pq_w4a8_linear_group_workspace_size(1, 4096, 5) == 0


def test_workspace_size_rules():
    lib = _lib.load()
    for m in (1, 4, 16, 3072):
        for n, k in ((1024, 4096), (4096, 4096), (12288, 4096), (4096, 12288)):
            assert lib.pq_w4a8_workspace_size(m, n, k, 128) == 0        # no inter-workgroup exchange
    # decode (m * k <= 8192, or m <= 2 for k >= 8192): rotated rows (fp32 bound) + per-group absmax
    def split(m, k):
        return (m * k * 4 + 255) // 256 * 256 + m * (k // 128) * 4
    assert lib.pq_w4a8_linear_workspace_size(1, 4096, 4096, 8) == split(1, 4096)
    assert lib.pq_w4a8_linear_workspace_size(1, 4096, 12288, 16) == split(1, 12288)
    assert lib.pq_w4a8_linear_workspace_size(2, 4096, 4096, 8) == split(2, 4096)
    assert lib.pq_w4a8_linear_workspace_size(2, 4096, 12288, 8) == split(2, 12288)
    # rows of k >= 4096 past that, up to 64 tokens: rotated rows and int8 codes, then group maxima
    # and token scales
    def split3(m, k):
        return (m * k * 4 + 255) // 256 * 256 + (m * k + 255) // 256 * 256 + m * (k // 128) * 4 + m * 4
    assert lib.pq_w4a8_linear_workspace_size(3, 4096, 12288, 8) == split3(3, 12288)
    assert lib.pq_w4a8_linear_workspace_size(5, 4096, 12288, 8) == split3(5, 12288)
    assert lib.pq_w4a8_linear_workspace_size(16, 4096, 12288, 8) == split3(16, 12288)
    assert lib.pq_w4a8_linear_workspace_size(32, 4096, 12288, 8) == split3(32, 12288)
    assert lib.pq_w4a8_linear_group_workspace_size(16, 8192, 2) == 2 * split3(16, 8192)
    assert lib.pq_w4a8_linear_workspace_size(4, 4096, 4096, 8) == split3(4, 4096)
    assert lib.pq_w4a8_linear_workspace_size(3, 4096, 4096, 8) == split3(3, 4096)
    assert lib.pq_w4a8_linear_workspace_size(17, 4096, 12288, 8) == split3(17, 12288)
    assert lib.pq_w4a8_linear_workspace_size(32, 4096, 4096, 8) == split3(32, 4096)
    assert lib.pq_w4a8_linear_workspace_size(33, 4096, 12288, 8) == split3(33, 12288)
    assert lib.pq_w4a8_linear_workspace_size(64, 4096, 4096, 8) == split3(64, 4096)
    # otherwise the row path holds xq and xscale
    assert lib.pq_w4a8_linear_workspace_size(65, 4096, 12288, 8) == 65 * 12288 + 260
    assert lib.pq_w4a8_linear_workspace_size(65, 4096, 4096, 8) == 65 * 4096 + 260
    assert lib.pq_w4a8_linear_workspace_size(5, 4096, 2048, 8) == 5 * 2048 + 20
    assert lib.pq_w4a8_linear_workspace_size(3, 64, 100, 8) == 0       # invalid shape -> 0


def test_status_names_and_error_type():
    with pytest.raises(_lib.PQError, match="PQ_ERR_ARG"):
        _lib.check(1, "x")
    _lib.check(0, "x")


def test_linear_group_rmsnorm_argument_checks():
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    mem = (_lib.LinearMember * 1)()
    mem[0] = _lib.LinearMember(256, 256, None, 256, 256, None, 256, 64)
    args = dict(count=1, bias_dtype=0, y_dtype=2, m=1, k=4096, krot=8, flags=3, ws=p, wsb=1 << 20, stream=None)

    def call(x=p, res=None, w=p, eps=1e-6, h=None, s=None, dt=2, **kw):
        a = dict(args, **kw)
        return lib.pq_w4a8_linear_group_rmsnorm(x, res, w, eps, h, s, dt, mem, a["count"], a["bias_dtype"],
                                                a["y_dtype"], a["m"], a["k"], a["krot"], a["flags"], a["ws"],
                                                a["wsb"], a["stream"])

    assert call(eps=-1.0) == 1 and "eps" in _err(lib)
    assert call(w=None) == 1 and "norm_weight" in _err(lib)
    assert call(res=ctypes.c_void_p(258)) == 1 and "residual" in _err(lib)
    assert call(s=p) == 1 and "sum_out" in _err(lib)
    assert call(dt=7) == 2
    assert call(m=0) == 0   # empty input: no-op


def test_w4a16_argument_checks():
    lib = _lib.load()
    p = ctypes.c_void_p(256)

    def gemm(x=p, m=4, n=64, k=256, gs=128, yd=2):
        return lib.pq_w4a16_gemm(x, p, p, None, 0, p, yd, m, n, k, gs, None)

    assert gemm(gs=64) == 2 and "group_size" in _err(lib)
    assert gemm(n=60) == 1
    assert gemm(k=200) == 1
    assert gemm(yd=9) == 2
    assert gemm(x=ctypes.c_void_p(258)) == 1 and "aligned" in _err(lib)
    assert gemm(x=None) == 1 and "null" in _err(lib)
    assert gemm(m=1 << 20, k=1 << 11) == 1   # 2*m*k reaches 2^31
    assert gemm(m=0) == 0                     # empty input: no-op
    assert lib.pq_w4a16_prepack(p, p, p, p, p, 256, 64, 64, None) == 2
    assert lib.pq_w4a16_prepack(p, p, p, p, p, 100, 64, 128, None) == 1
    assert lib.pq_w4a16_prepack(p, None, p, p, p, 256, 64, 128, None) == 1

    def linear(m=1, k=4096, krot=8, flags=0, ws=None, wsb=0, xd=1):
        return lib.pq_w4a16_linear(p, xd, p, p, None, p, p, None, 0, p, 1, m, 4096, k, krot, flags, ws, wsb, None)

    assert linear(krot=0) == 2
    assert linear(flags=2) == 1 and "flags" in _err(lib)   # the fp16 rounding of the rotation is implied
    assert linear(xd=5) == 2
    assert linear(k=32768) == 1
    assert linear(m=0) == 0
    need1 = lib.pq_w4a16_linear_workspace_size(1, 4096)
    assert need1 == 2 * 4096 + 256                           # fp16 row + the split rotation's group maxima,
    assert lib.pq_w4a16_linear_workspace_size(1, 1152) == 2560          # the sum rounded up to 256 bytes
    assert lib.pq_w4a16_linear_workspace_size(3, 384) == 2560
    need64 = lib.pq_w4a16_linear_workspace_size(64, 4096)
    assert need64 == 64 * 4096 * 2
    assert lib.pq_w4a16_linear_workspace_size(0, 4096) == 0
    assert linear(m=64) == 4 and "workspace" in _err(lib)
    assert linear(m=64, ws=p, wsb=need64 - 1) == 4
    assert linear(m=64, ws=ctypes.c_void_p(272), wsb=need64) == 4


def test_rotate_mxfp4_argument_checks():
    lib = _lib.load()
    p = ctypes.c_void_p(256)

    def call(x=p, q=p, s=p, rows=4, h=256, krot=8, gs=128, dt=2):
        return lib.pq_rotate_mxfp4(x, q, s, p, p, None, rows, h, krot, gs, dt, None)

    assert call(gs=32) == 2 and "group_size" in _err(lib)
    assert call(krot=3) == 2
    assert call(h=200) == 1
    assert call(dt=9) == 2
    assert call(q=ctypes.c_void_p(258)) == 1 and "aligned" in _err(lib)
    assert call(s=None) == 1 and "null" in _err(lib)
    assert call(rows=0) == 0


def test_linear_group_fused_argument_checks():
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    mem = (_lib.LinearMember * 1)()
    mem[0] = _lib.LinearMember(256, 256, None, 256, 256, None, 256, 64)
    args = dict(count=1, bias_dtype=0, y_dtype=2, m=1, k=4096, krot=8, flags=3, ws=p, wsb=1 << 20, stream=None)

    def call(mode, x2=p, w=None, eps=0.0, h=None, s=None, **kw):
        a = dict(args, **kw)
        return lib.pq_w4a8_linear_group_fused(p, x2, w, eps, mode, h, s, 2, mem, a["count"], a["bias_dtype"],
                                              a["y_dtype"], a["m"], a["k"], a["krot"], a["flags"], a["ws"], a["wsb"],
                                              a["stream"])

    assert call(7) == 1 and "mode" in _err(lib)
    assert call(_lib.PQ_PRO_ADD, x2=None) == 1 and "x2" in _err(lib)
    assert call(_lib.PQ_PRO_SWIGLU, x2=None) == 1
    assert call(_lib.PQ_PRO_ADD, h=p) == 1 and "h_out" in _err(lib)
    assert call(_lib.PQ_PRO_SWIGLU, s=p) == 1 and "sum_out" in _err(lib)
    assert call(_lib.PQ_PRO_RMSNORM, w=None, eps=1e-6) == 1 and "norm_weight" in _err(lib)
    assert call(_lib.PQ_PRO_ADD, x2=ctypes.c_void_p(258)) == 1 and "aligned" in _err(lib)
    assert call(_lib.PQ_PRO_SWIGLU, m=0) == 0


def test_w4a16_group_workspace_rule():
    lib = _lib.load()
    for m, k in ((1, 4096), (16, 12288), (300, 4096), (1, 1152), (3, 384), (1, 384)):
        one = lib.pq_w4a16_linear_workspace_size(m, k)
        assert one > 0 and one % 256 == 0     # every member's block starts 256-byte aligned
        for count in (1, 2, 3, 4):
            assert lib.pq_w4a16_linear_group_workspace_size(m, k, count) == count * one
    assert lib.pq_w4a16_linear_group_workspace_size(1, 4096, 0) == 0
    assert lib.pq_w4a16_linear_group_workspace_size(1, 4096, 5) == 0


def test_split_path_rule():
    lib = _lib.load()
    assert lib.pq_w4a8_linear_split_path(1, 4096) == 1
    assert lib.pq_w4a8_linear_split_path(3, 4096) == 1   # three tokens: the three launches
    assert lib.pq_w4a8_linear_split_path(1, 12288) == 1
    assert lib.pq_w4a8_linear_split_path(4, 4096) == 1
    assert lib.pq_w4a8_linear_split_path(5, 2048) == 0   # short rows: the row kernel
    # long rows: the split pair up to 2 tokens, then the three-launch split path (never the row kernel)
    assert lib.pq_w4a8_linear_split_path(2, 12288) == 1
    assert lib.pq_w4a8_linear_split_path(4, 12288) == 1
    assert lib.pq_w4a8_linear_split_path(4, 8192) == 1
    assert lib.pq_w4a8_linear_split_path(4, 16384) == 1
    assert lib.pq_w4a8_linear_split_path(5, 12288) == 1    # long rows: the three-launch split path
    assert lib.pq_w4a8_linear_split_path(16, 8192) == 1
    assert lib.pq_w4a8_linear_split_path(17, 12288) == 1
    assert lib.pq_w4a8_linear_split_path(32, 16384) == 1
    assert lib.pq_w4a8_linear_split_path(33, 12288) == 1
    assert lib.pq_w4a8_linear_split_path(64, 16384) == 1
    assert lib.pq_w4a8_linear_split_path(65, 12288) == 0
    assert lib.pq_w4a8_linear_split_path(16, 4096) == 1
    assert lib.pq_w4a8_linear_split_path(64, 4096) == 1
    assert lib.pq_w4a8_linear_split_path(65, 4096) == 0
    assert lib.pq_w4a8_linear_split_path(2, 4096) == 1
    assert lib.pq_w4a8_linear_split_path(4, 6144) == 1
    assert lib.pq_w4a8_linear_split_path(3, 3968) == 0
    assert lib.pq_w4a8_linear_split_path(0, 4096) == 0


def test_rotate_rows_argument_checks():
    lib = _lib.load()
    p = ctypes.c_void_p(256)

    def call(x=p, dt=2, out=p, mxs=None, rows=4, h=256, krot=8, mode=0):
        return lib.pq_rotate_rows(x, dt, p, p, None, out, mxs, rows, h, krot, mode, None)

    assert call(h=192) == 1
    assert call(krot=17) == 2
    assert call(dt=5) == 2
    assert call(mode=3) == 1 and "out_mode" in _err(lib)
    assert call(mode=1) == 1 and "null" in _err(lib)              # MXFP4 needs the scale buffer
    assert call(x=ctypes.c_void_p(264)) == 1 and "aligned" in _err(lib)
    assert call(rows=0) == 0


def test_w4a16_linear_group_argument_checks():
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    mem = (_lib.LinearMember * 5)()
    for i in range(5):
        mem[i] = _lib.LinearMember(256, 256, None, 256, 256, None, 256, 64)
    call = lambda members, count, m=2, k=1024, ws=p, wsb=1 << 20: lib.pq_w4a16_linear_group(  # noqa: E731
        p, 1, members, count, 0, 1, m, k, 8, 1, ws, wsb, None)
    assert call(mem, 0) == 1 and "count" in _err(lib)
    assert call(mem, 5) == 1
    assert call(None, 2) == 1 and "member table" in _err(lib)
    mem[1].n = 40
    assert call(mem, 2) == 1
    mem[1].n = 64
    assert call(mem, 2, k=1000) == 1
    assert call(mem, 2, m=0) == 0                                  # empty input: nothing to do
    mem[0].rot_idx = None
    assert call(mem, 2) == 1 and "member 0: null pointer" in _err(lib)
    mem[0].rot_idx = 256
    mem[1].wpack = 264                                             # 8-byte aligned only
    assert call(mem, 2) == 1 and "member 1: misaligned" in _err(lib)
    mem[1].wpack = 256
    assert call(mem, 2, wsb=16) == 4 and "workspace" in _err(lib)  # workspace too small
    assert call(mem, 2, ws=ctypes.c_void_p(272)) == 4              # workspace not 256-byte aligned


def test_rotate_backward_argument_checks():
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    ws = lib.pq_rotate_backward_workspace_size(100, 256, 8)
    assert ws == 7 * (8 * 128 + 256) * 4                                 # ceil(100 / 16) row tiles
    assert lib.pq_rotate_backward_workspace_size(10 ** 6, 256, 8) == 64 * (8 * 128 + 256) * 4   # capped at 64
    assert lib.pq_rotate_backward_workspace_size(0, 256, 8) == 0
    call = lambda rows=4, h=256, krot=8, gs=128, dt=1, sc=None, gsc=None, w=p, wb=1 << 20: lib.pq_rotate_backward(  # noqa: E731
        p, p, p, p, gsc, p, p, sc, rows, h, krot, gs, dt, w, wb, None)
    assert call(gs=32) == 2 and "group_size" in _err(lib)
    assert call(krot=3) == 2 and "KROT" in _err(lib)
    assert call(h=200) == 1 and "divisible" in _err(lib)
    assert call(dt=7) == 2
    assert call(sc=p) == 1 and "grad_scales" in _err(lib)
    assert call(gsc=p) == 1 and "grad_scales" in _err(lib)
    assert call(wb=16) == 4 and "workspace" in _err(lib)
    assert call(w=None) == 4


def test_split_path_python_rule_matches_library():
    """ops.split_path (the Python form torch.compile traces) agrees with pq_w4a8_linear_split_path."""
    from alpamayo_amd import ops

    lib = _lib.load()
    for k in range(128, 16384 + 1, 128):
        for m in list(range(0, 40)) + [47, 48, 63, 64, 65, 96, 1000, 3072]:
            assert ops.split_path(m, k) == bool(lib.pq_w4a8_linear_split_path(m, k)), (m, k)
    assert ops.split_path(1, 16384 + 128) == bool(lib.pq_w4a8_linear_split_path(1, 16384 + 128))
    # depths that are not a multiple of 128 take neither split path, in either form
    for k in (8200, 12290, 4100, 100):
        for m in (1, 2, 3, 17, 32):
            assert not ops.split_path(m, k) and not lib.pq_w4a8_linear_split_path(m, k), (m, k)

