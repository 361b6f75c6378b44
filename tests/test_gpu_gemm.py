"""GPU parity of the W4A8 GEMM kernels and the AWQ prepack against the oracle.

Bar: per-group int32 partials bit-exact; outputs within 1e-2 relative
(Frobenius) of the float64 oracle and within a few bf16 ulps elementwise.
"""

import zlib

import numpy as np
import pytest
import torch

import alpamayo_amd  # noqa: F401
from alpamayo_amd import workloads
from oracle import gemm as ogemm
from oracle import packing as opack
from tests.gpu_util import assert_bf16_close, to_np

pytestmark = pytest.mark.gpu


def _case(M, N, K, seed):
    g = workloads.generator(seed)
    w = workloads.weights(N, K, g, keep_codes=True)
    xq = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
    xs = (0.01 + torch.rand(M, generator=g)).float()
    return w, xq, xs


def _prepack(w):
    return torch.ops.paroquant.w4a8_prepack(w.awq_qweight.cuda(), w.awq_scales.cuda(), w.awq_qzeros.cuda())


@pytest.mark.parametrize("N,K", [(16, 128), (48, 384), (1024, 4096), (128, 12288)])
def test_prepack_bit_exact(N, K):
    w, _, _ = _case(1, N, K, N + K)
    wp, wm = _prepack(w)
    ref_p, ref_m = opack.prepack_kernel_layout(w.codes.numpy(), w.awq_scales.numpy(), w.zeros.numpy())
    np.testing.assert_array_equal(to_np(wp), ref_p)
    np.testing.assert_array_equal(to_np(wm).view(np.uint32), ref_m)


SHAPES = [(1, 16, 128), (3, 64, 256), (16, 1024, 4096), (4, 4096, 4096), (1, 1024, 4096), (17, 128, 256),
          (33, 48, 256), (130, 256, 512), (257, 384, 1024), (64, 1024, 12288), (200, 1552, 384),
          # decode GEMM with two column tiles per workgroup: 384 tiles (between one and two rounds of one)
          (8, 6144, 1024),
          # decode GEMM on two to four row blocks of 16 (17-64 rows), one and two column tiles per workgroup
          (32, 4096, 1024), (24, 6144, 512), (40, 6144, 1024), (64, 4096, 4096), (49, 1024, 12288)]
# prefill tiling: 192 x 256 workgroup tiles once there are >= 256 of them, else 128 x 256 when 128-256 of
# those, else 128 x 128 or 64 x 128.
# These reach the big tiles with an odd group count, ragged M and a partial last column tile.
BIG_TILE_SHAPES = [(1500, 8176, 384), (3000, 4112, 256),
                   # 128 x 256 tiles (half to one round of them): ragged M, a partial last column tile
                   (1300, 4096, 384), (2000, 4080, 256)]


@pytest.mark.parametrize("M,N,K", SHAPES + BIG_TILE_SHAPES)
def test_partials_bit_exact(M, N, K):
    print(f"partials M={M} N={N} K={K}", flush=True)
    w, xq, _ = _case(M, N, K, zlib.crc32(f"p{M}-{N}-{K}".encode()))
    wp, wm = _prepack(w)
    P = torch.ops.paroquant.w4a8_gemm_partials(xq.cuda(), wp, wm)
    ref = ogemm.group_partials(xq.numpy(), w.codes.numpy(), w.zeros.numpy())
    np.testing.assert_array_equal(to_np(P), ref)


@pytest.mark.parametrize("M,N,K", SHAPES + BIG_TILE_SHAPES)
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_gemm_matches_oracle(M, N, K, out_dtype):
    print(f"gemm M={M} N={N} K={K} {out_dtype}", flush=True)
    w, xq, xs = _case(M, N, K, zlib.crc32(f"g{M}-{N}-{K}".encode()))
    wp, wm = _prepack(w)
    y = torch.ops.paroquant.w4a8_gemm(xq.cuda(), xs.cuda(), wp, wm, None, out_dtype)
    ref = ogemm.w4a8_linear(xq.numpy(), xs.numpy(), w.codes.numpy(), w.awq_scales.numpy(), w.zeros.numpy())
    assert y.dtype == out_dtype and y.shape == (M, N)
    assert_bf16_close(to_np(y), ref)


def test_gemm_bias_and_repeatability():
    M, N, K = 5, 1024, 4096
    w, xq, xs = _case(M, N, K, 99)
    wp, wm = _prepack(w)
    bias = torch.randn(N).to(torch.bfloat16)
    y1 = torch.ops.paroquant.w4a8_gemm(xq.cuda(), xs.cuda(), wp, wm, bias.cuda(), torch.bfloat16)
    y2 = torch.ops.paroquant.w4a8_gemm(xq.cuda(), xs.cuda(), wp, wm, bias.cuda(), torch.bfloat16)
    assert torch.equal(y1, y2)                       # fixed-order sums: repeatable bit for bit
    ref = ogemm.w4a8_linear(xq.numpy(), xs.numpy(), w.codes.numpy(), w.awq_scales.numpy(), w.zeros.numpy(),
                            bias.float().numpy())
    assert_bf16_close(to_np(y1), ref)


@pytest.mark.parametrize("M,N,K", [(5, 1024, 4096), (1500, 8176, 384)])
def test_gemm_bias_f32_out(M, N, K):
    w, xq, xs = _case(M, N, K, 7 + M)
    wp, wm = _prepack(w)
    bias = torch.randn(N).half()
    y = torch.ops.paroquant.w4a8_gemm(xq.cuda(), xs.cuda(), wp, wm, bias.cuda(), torch.float32)
    ref = ogemm.w4a8_linear(xq.numpy(), xs.numpy(), w.codes.numpy(), w.awq_scales.numpy(), w.zeros.numpy(),
                            bias.float().numpy())
    assert_bf16_close(to_np(y), ref)


@pytest.mark.parametrize("M,N,K", [(5, 1024, 4096), (200, 1552, 384), (1500, 8176, 384)])
def test_gemm_16bit_outputs_are_rounded_f32(M, N, K):
    """bf16 and fp16 outputs are the float32 output rounded to nearest even (torch's conversion), bit for bit,
    on the decode kernel, the small-tile and the 192 x 256 prefill kernels: every output type computes the same
    float32 value and converts it last (v_cvt_pk_bf16_f32 / v_cvt_f16_f32)."""
    w, xq, xs = _case(M, N, K, 11 + M)
    wp, wm = _prepack(w)
    bias = torch.randn(N, generator=workloads.generator(12 + M)).half().cuda()
    y32 = torch.ops.paroquant.w4a8_gemm(xq.cuda(), xs.cuda(), wp, wm, bias, torch.float32)
    for dt in (torch.bfloat16, torch.float16):
        y = torch.ops.paroquant.w4a8_gemm(xq.cuda(), xs.cuda(), wp, wm, bias, dt)
        assert torch.equal(y.view(torch.int16), y32.to(dt).view(torch.int16)), dt


def test_gemm_extreme_operands_exact():
    """All codes 15 vs zero 0 and activations -128/127: the largest partials are still exact."""
    M, N, K = 20, 32, 256
    G = K // 128
    codes = torch.full((N, K), 15, dtype=torch.int32)
    zeros = torch.zeros(G, N, dtype=torch.int32)
    zeros[1] = 15
    w = workloads.Weights(workloads.pack_awq(codes.t().contiguous()), torch.full((G, N), 0.02).half(),
                          workloads.pack_awq(zeros), codes.to(torch.uint8), zeros)
    xq = torch.full((M, K), 127, dtype=torch.int8)
    xq[::2] = -128
    wp, wm = _prepack(w)
    for m in (M, 16):
        P = torch.ops.paroquant.w4a8_gemm_partials(xq[:m].cuda(), wp, wm)
        ref = ogemm.group_partials(xq[:m].numpy(), codes.numpy(), zeros.numpy())
        np.testing.assert_array_equal(to_np(P), ref)


def test_gemm_empty_and_errors():
    w, xq, xs = _case(4, 64, 256, 5)
    wp, wm = _prepack(w)
    y = torch.ops.paroquant.w4a8_gemm(xq[:0].cuda(), xs[:0].cuda(), wp, wm, None, torch.bfloat16)
    assert y.shape == (0, 64)
    with pytest.raises(RuntimeError, match="xq must be int8"):
        torch.ops.paroquant.w4a8_gemm(xq[:, :128].cuda(), xs.cuda(), wp, wm, None, torch.bfloat16)
    with pytest.raises(RuntimeError, match="awq_scales"):
        torch.ops.paroquant.w4a8_prepack(w.awq_qweight.cuda(), w.awq_scales.float().cuda(), w.awq_qzeros.cuda())


# The prefill GEMM at the full Qwen3-8B depths with 192 x 256 tiles (>= 256 tiles): q/o (4096 x 4096), the
# q/k/v group's concatenated columns (6144 x 4096), gate/up's (24576 x 4096 would need 9.6 GB of partials;
# 12288 x 4096 has the same tiling per column block) and down (4096 x 12288); partials checked bit for bit on
# rows spread over every row tile position.
@pytest.mark.parametrize("N,K", [(4096, 4096), (6144, 4096), (12288, 4096), (4096, 12288)])
def test_partials_full_depth_big_tiles_row_subset(N, K):
    M = 3072
    print(f"partials full depth M={M} N={N} K={K}", flush=True)
    w, xq, _ = _case(M, N, K, zlib.crc32(f"fd{N}-{K}".encode()))
    wp, wm = _prepack(w)
    rng = np.random.default_rng(N + K)
    rows = np.unique(np.concatenate([[0, 1, 191, 192, 383, 1535, 3071], rng.integers(0, M, 9)]))
    P = torch.ops.paroquant.w4a8_gemm_partials(xq.cuda(), wp, wm)
    got = to_np(P[torch.from_numpy(rows).cuda()])
    del P
    ref = ogemm.group_partials(xq.numpy()[rows], w.codes.numpy(), w.zeros.numpy())
    np.testing.assert_array_equal(got, ref)
