"""Parity of what the production W4A8 linear paths multiply (pq_w4a8_linear_group_intermediates).

The linear entry points pick one of three launch sequences by token count and row length: the split pair
(split rotation, then a decode GEMM that derives the token scales and int8 codes itself: in registers at one
and two tokens, into LDS otherwise),
the three-launch long-row path (split rotation, quant_split_kernel, decode GEMM on int8 A) and the row
rotate+quant kernel followed by the decode GEMM (up to 64 rows) or the prefill GEMM (tile-pair form on its big
tiles).  The intermediates entry point runs the same launches with the GEMM in its partials form and returns the
int8 codes and token scales that GEMM used and its int32 per-group partials.  Checked here, against the oracle,
for every path, every prologue (none, RMSNorm, residual add, SwiGLU), single linears and groups, on the
Qwen3-8B decoder-layer shapes at 1-64 tokens and at prefill sizes:

  - int8 codes: >= 99.9 % identical to the oracle's per-token quantization (vLLM scaled_int8_quant semantics,
    as invoked before the Marlin GEMM at paroquant_marlin_w4a8.py:319-333) of the oracle's rotation of the
    same rows, and never more than 1 LSB apart;
  - token scales: absmax / 127 within rtol 1e-6;
  - int32 partials: bit-exact against the exact integer partials of the GPU's own codes (the accumulators of
    the Marlin GEMM, same call site).

The rows fed to the oracle's rotation are what the kernel rotated: x for the plain group, the h / s the fused
prologue wrote (h within 1 ulp and s exact against their own oracles, test_gpu_rmsnorm.py /
test_gpu_prologue.py).
"""

import functools
import zlib

import numpy as np
import pytest
import torch

import alpamayo_amd  # noqa: F401
from alpamayo_amd import _lib, ops, workloads
from oracle import gemm as ogemm
from oracle import quant as oquant
from oracle import rotation as orot
from tests.gpu_util import assert_codes_close, to_np
from tests.test_gpu_group import _members

pytestmark = pytest.mark.gpu

# The layer's calls: q/k/v over the attention input, o, gate/up over the MLP input, down over the activation.
LAYOUTS = {"qkv": (4096, (4096, 1024, 1024)), "o": (4096, (4096,)), "gateup": (4096, (12288, 12288)),
           "down": (12288, (4096,))}


@functools.lru_cache(maxsize=None)
def _layer_members(ns, K, krot=8):
    """Members for a (columns, depth) layout, built once per test module (their weights do not depend on M)."""
    return _members(ns, K, krot, zlib.crc32(f"imd-members-{ns}-{K}-{krot}".encode()), with_bias=False)


def _check(mbs, rows_np, codes, xscale, parts, flags, rows=None):
    """Codes / scales against the oracle on rows_np, partials bit-exact on the GPU's codes (row subset)."""
    codes_np, xs_np = to_np(codes), to_np(xscale)
    sel = np.arange(codes_np.shape[1]) if rows is None else rows
    for i, mb in enumerate(mbs):
        v = orot.rotate_path_f32(rows_np[sel], mb["pairs"].numpy(), mb["c"], mb["s"], mb["scales"].cpu().numpy(),
                                 128, *flags)
        qref, sref = oquant.quant_int8_per_token(v)
        assert_codes_close(codes_np[i][sel], qref)
        np.testing.assert_allclose(xs_np[i][sel], sref, rtol=1e-6, atol=0)
        got = to_np(parts[i][torch.from_numpy(sel).cuda()]) if rows is not None else to_np(parts[i])
        ref = ogemm.group_partials(codes_np[i][sel], mb["spec"].w.codes.numpy(), mb["spec"].w.zeros.numpy())
        np.testing.assert_array_equal(got, ref)


def _run(mbs, x, krot, flags, **kw):
    return ops.w4a8_linear_group_intermediates(
        x, [m["rot_idx"] for m in mbs], [m["rot_cs"] for m in mbs], [m["scales"] for m in mbs], krot,
        [m["wp"] for m in mbs], [m["wm"] for m in mbs], flags[0], flags[1], **kw)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 16, 17, 32, 33, 48, 64])
@pytest.mark.parametrize("layout", list(LAYOUTS))
def test_plain_group_intermediates(M, layout):
    K, ns = LAYOUTS[layout]
    print(f"intermediates plain {layout} M={M} K={K} ns={ns} split={ops.split_path(M, K)}", flush=True)
    seed = zlib.crc32(f"imd{layout}-{M}".encode())
    krot, flags = 8, (True, True)
    mbs = _layer_members(ns, K, krot)
    x = workloads.activations(M, K, workloads.generator(seed + 1)).cuda()
    codes, xscale, parts, _, _ = _run(mbs, x, krot, flags)
    assert codes.shape == (len(ns), M, K) and xscale.shape == (len(ns), M)
    _check(mbs, to_np(x), codes, xscale, parts, flags)


@pytest.mark.parametrize("M,K,ns", [(1, 4096, (4096, 1024)), (2, 4096, (1024,)), (2, 12288, (4096,)),
                                    (5, 12288, (1024,)), (20, 8192, (1024, 64)), (9, 4096, (1024,)),
                                    (6, 2048, (1024,))])
def test_unrounded_rows_intermediates(M, K, ns):
    """flags (False, False): no fp16 rounding of the input or of the rotated rows (the fp32 operand of the
    quantizing prologue, AQ = 2, and of quant_split_kernel)."""
    print(f"intermediates fp32 rows M={M} K={K} ns={ns}", flush=True)
    seed = zlib.crc32(f"imdf{M}-{K}-{ns}".encode())
    krot, flags = 8, (False, False)
    mbs = _layer_members(ns, K, krot)
    x = workloads.activations(M, K, workloads.generator(seed + 1)).cuda()
    codes, xscale, parts, _, _ = _run(mbs, x, krot, flags)
    _check(mbs, to_np(x), codes, xscale, parts, flags)


@pytest.mark.parametrize("M", [1, 2, 4, 16, 32, 48, 64])
@pytest.mark.parametrize("layout", ["qkv", "gateup"])
def test_rmsnorm_prologue_intermediates(M, layout):
    K, ns = LAYOUTS[layout]
    print(f"intermediates rmsnorm {layout} M={M}", flush=True)
    seed = zlib.crc32(f"imdr{layout}-{M}".encode())
    krot, flags = 8, (True, True)
    mbs = _layer_members(ns, K, krot)
    g = workloads.generator(seed + 1)
    x, r = workloads.activations(M, K, g).cuda(), workloads.activations(M, K, g).cuda()
    w = (0.8 + 0.4 * torch.rand(K, generator=g)).to(torch.bfloat16).cuda()
    codes, xscale, parts, h, s = _run(mbs, x, krot, flags, x2=r, norm_weight=w, eps=1e-6, mode=_lib.PQ_PRO_RMSNORM,
                                      return_h=True, return_sum=True)
    assert torch.equal(s, x + r)
    _check(mbs, to_np(h), codes, xscale, parts, flags)


@pytest.mark.parametrize("M,K,ns", [(4, 8192, (1024,)), (17, 12288, (4096,)), (13, 8192, (1024, 64)),
                                   (40, 12288, (4096,)), (64, 8192, (1024, 64))])
def test_rmsnorm_prologue_long_rows(M, K, ns):
    """The RMSNorm prologue on the three-launch long-row path."""
    print(f"intermediates rmsnorm long rows M={M} K={K} ns={ns}", flush=True)
    seed = zlib.crc32(f"imdrl{M}-{K}".encode())
    krot, flags = 8, (True, True)
    mbs = _layer_members(ns, K, krot)
    g = workloads.generator(seed + 1)
    x = workloads.activations(M, K, g).cuda()
    w = (0.8 + 0.4 * torch.rand(K, generator=g)).to(torch.bfloat16).cuda()
    codes, xscale, parts, h, _ = _run(mbs, x, krot, flags, norm_weight=w, eps=1e-6, mode=_lib.PQ_PRO_RMSNORM,
                                      return_h=True)
    _check(mbs, to_np(h), codes, xscale, parts, flags)


@pytest.mark.parametrize("M", [1, 2, 4, 16, 32, 48, 64])
def test_add_prologue_intermediates(M):
    K, ns = LAYOUTS["qkv"]
    print(f"intermediates add qkv M={M}", flush=True)
    seed = zlib.crc32(f"imda{M}".encode())
    krot, flags = 8, (True, True)
    mbs = _layer_members(ns, K, krot)
    g = workloads.generator(seed + 1)
    x, r = workloads.activations(M, K, g).cuda(), workloads.activations(M, K, g).cuda()
    codes, xscale, parts, _, s = _run(mbs, x, krot, flags, x2=r, mode=_lib.PQ_PRO_ADD, return_sum=True)
    assert torch.equal(s, x + r)
    _check(mbs, to_np(s), codes, xscale, parts, flags)


@pytest.mark.parametrize("M,K", [(1, 12288), (2, 12288), (3, 12288), (16, 12288), (17, 12288), (24, 12288),
                                 (32, 12288), (32, 16384), (2, 4096), (16, 4096), (1, 16384), (1, 8320),
                                 (48, 12288), (64, 12288)])
def test_swiglu_prologue_intermediates(M, K):
    """down_proj's input silu(gate) * up: the split pair, the long-row path up to 64 tokens, the row path.
    At one token the GEMM quantizes A in registers: K = 16384 takes all 128 group maxima, K = 8320 (65
    groups) leaves the last batch part past K."""
    ns = (4096,)
    print(f"intermediates swiglu down M={M} K={K}", flush=True)
    seed = zlib.crc32(f"imdg{M}-{K}".encode())
    krot, flags = 8, (True, True)
    mbs = _layer_members(ns, K, krot)
    g = workloads.generator(seed + 1)
    gate, up = workloads.activations(M, K, g).cuda(), workloads.activations(M, K, g).cuda()
    codes, xscale, parts, h, _ = _run(mbs, gate, krot, flags, x2=up, mode=_lib.PQ_PRO_SWIGLU, return_h=True)
    _check(mbs, to_np(h), codes, xscale, parts, flags)


@pytest.mark.parametrize("M,K,ns", [
    (300, 4096, (4096, 1024, 1024)),     # 128 x 256 / 128 x 128 tiles
    (1264, 4096, (4096, 1024, 1024)),    # the ragged batch's total: 128 x 256 tiles (tile-pair form)
    (1264, 12288, (4096,)),
    (3072, 4096, (4096, 1024, 1024)),    # q on 192 x 256 tiles, k/v on 128 x 256 tiles (tile-pair form)
    (3072, 12288, (4096,)),              # down at full depth, 192 x 256 tiles
    (2053, 512, (1040, 16)),             # row blocks sized to fill rounds, with a remainder row
])
def test_prefill_intermediates_row_subset(M, K, ns):
    """Prefill: the row rotate+quant kernel and the prefill GEMM in the form production runs (tile pairs on the
    big tiles), checked on rows spread over every row-tile position."""
    print(f"intermediates prefill M={M} K={K} ns={ns}", flush=True)
    seed = zlib.crc32(f"imdp{M}-{K}-{ns}".encode())
    krot, flags = 8, (True, True)
    mbs = _layer_members(ns, K, krot)
    x = workloads.activations(M, K, workloads.generator(seed + 1)).cuda()
    codes, xscale, parts, _, _ = _run(mbs, x, krot, flags)
    rng = np.random.default_rng(M + K)
    rows = np.unique(np.concatenate([[0, 1, 31, 32, 127, 128, 191, 192, 255, M // 2, M - 1],
                                     rng.integers(0, M, 6)]))
    rows = rows[rows < M]
    _check(mbs, to_np(x), codes, xscale, parts, flags, rows=rows)
    # every row's codes reach +-127 (the token scale is the row's absmax / 127)
    assert np.all(np.abs(to_np(codes).astype(np.int32)).max(axis=2) == 127)


def test_intermediates_match_the_linear_outputs():
    """The intermediates are those of the product path: the bf16 outputs of paroquant::w4a8_linear_group equal
    the epilogue applied to the returned partials and scales (float64, within a bf16 rounding)."""
    K, ns = LAYOUTS["qkv"]
    for M in (1, 3, 20, 300):
        mbs = _layer_members(ns, K)
        x = workloads.activations(M, K, workloads.generator(4243 + M)).cuda()
        codes, xscale, parts, _, _ = _run(mbs, x, 8, (True, True))
        outs = torch.ops.paroquant.w4a8_linear_group(
            x, [m["rot_idx"] for m in mbs], [m["rot_cs"] for m in mbs], [m["scales"] for m in mbs], 8,
            [m["wp"] for m in mbs], [m["wm"] for m in mbs], [None] * len(ns), True, True, torch.bfloat16)
        for i, (mb, y) in enumerate(zip(mbs, outs)):
            P = to_np(parts[i]).astype(np.float64)                                   # [M, G, N]
            s = mb["spec"].w.awq_scales.numpy().astype(np.float64)                  # [G, N]
            ref = np.einsum("mgn,gn->mn", P, s) * to_np(xscale[i]).astype(np.float64)[:, None]
            got = to_np(y).astype(np.float64)
            assert np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-6 * np.abs(ref).max())


def test_intermediates_argument_errors():
    K, ns = 4096, (1024,)
    mbs = _layer_members(ns, K)
    x = workloads.activations(2, K, workloads.generator(78)).cuda()
    with pytest.raises(RuntimeError, match="mode"):
        _run(mbs, x, 8, (True, True), mode=9)
    with pytest.raises(RuntimeError, match="x2"):
        _run(mbs, x, 8, (True, True), mode=_lib.PQ_PRO_ADD)
