"""End-to-end GPU parity of the quantized-Linear modules (the reference's
RotateLinearInt4 / MarlinW4A8Linear / BF16RotateLinearWrapper call chain,
paroquant_marlin_w4a8.py:59-65, 314-333; rotation_linear.py:120-124) on the
benchmark configurations, against the oracle."""

import zlib

import numpy as np
import pytest
import torch

import alpamayo_amd  # noqa: F401
from alpamayo_amd import workloads
from alpamayo_amd.quantization import (
    BF16RotateLinearWrapper,
    MarlinW4A8Linear,
    RotateLinearInt4,
    WQLinear,
    convert_model_to_marlin_w4a8,
    pack_intweight,
)
from oracle import gemm as ogemm
from oracle import linear as olin
from oracle import quant as oquant
from oracle import rotation as orot
from tests.gpu_util import assert_bf16_close, assert_codes_close, packed_rotation, rel_fro, to_np

pytestmark = pytest.mark.gpu


def _oracle_linear(spec, x_bf16_np, rows=None):
    c, s = orot.cos_sin_table(spec.theta.numpy())
    xr = x_bf16_np if rows is None else x_bf16_np[rows]
    y, q, sx = olin.w4a8_rotate_linear(xr, spec.pairs.numpy(), c, s, spec.channel_scales.float().reshape(-1).numpy(),
                                       spec.w.codes.numpy(), spec.w.awq_scales.numpy(), spec.w.zeros.numpy())
    return y, q, sx


def test_config0_single_linear_m16():
    """Config 0: X bf16 [16, 4096] with 1% x20 outliers through one 4096->4096 linear."""
    spec = workloads.linear_spec("q_proj", 4096, 4096, workloads.generator(1000), keep_codes=True)
    x = workloads.activations(16, 4096, workloads.generator(1000 + 7))
    mod = workloads.build_module(spec, "cuda")
    y = mod(x.cuda())
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16 and y.shape == (16, 4096)
    ref, _, _ = _oracle_linear(spec, to_np(x))
    assert_bf16_close(to_np(y), ref)


@pytest.mark.parametrize("M", [1, 4, 16])
def test_config1_decode_all_seven_shapes(M):
    for i, (name, (N, K)) in enumerate(workloads.QWEN3_8B_LINEARS.items()):
        print(f"decode M={M} {name} N={N} K={K}", flush=True)
        spec = workloads.linear_spec(name, N, K, workloads.generator(1001 + 10 * i), keep_codes=True)
        x = workloads.activations(M, K, workloads.generator(2001 + 10 * i + M))
        y = workloads.build_module(spec, "cuda")(x.cuda())
        ref, _, _ = _oracle_linear(spec, to_np(x))
        assert_bf16_close(to_np(y), ref)


def test_config2_prefill_shapes_row_subset():
    """Config 2: M = 3072 through q (4096->4096), k (4096->1024) and down (12288->4096), rows checked on a subset."""
    rows = np.array([0, 5, 1500, 3071])
    for i, name in enumerate(["q_proj", "k_proj", "down_proj"]):
        N, K = workloads.QWEN3_8B_LINEARS[name]
        print(f"prefill M=3072 {name}", flush=True)
        spec = workloads.linear_spec(name, N, K, workloads.generator(1002 + i), keep_codes=True)
        x = workloads.activations(3072, K, workloads.generator(3002 + i))
        y = workloads.build_module(spec, "cuda")(x.cuda())
        ref, _, _ = _oracle_linear(spec, to_np(x), rows)
        assert_bf16_close(to_np(y)[rows], ref)


def test_config4_ragged_packed_batch():
    """Config 4: 8 requests of U{1..512} tokens packed without padding; per-row quant,
    so each request's rows equal a separate call on that request alone."""
    lens = workloads.ragged_lengths(8, workloads.generator(1004))
    offs = np.concatenate([[0], np.cumsum(lens)])
    N, K = workloads.QWEN3_8B_LINEARS["gate_proj"]
    spec = workloads.linear_spec("gate_proj", N, K, workloads.generator(1104), keep_codes=True)
    mod = workloads.build_module(spec, "cuda")
    x = workloads.activations(int(offs[-1]), K, workloads.generator(1204)).cuda()
    y = mod(x)
    for r in range(8):
        yr = mod(x[offs[r]:offs[r + 1]])
        assert rel_fro(to_np(yr), to_np(y[offs[r]:offs[r + 1]])) < 1e-2
    rows = np.array([0, int(offs[3]), int(offs[-1]) - 1])
    ref, _, _ = _oracle_linear(spec, to_np(x), rows)
    assert_bf16_close(to_np(y)[rows], ref)


def test_unfused_reference_chain_matches_fused():
    """rotation::rotate (fp16) -> MarlinW4A8Linear.forward (quant + GEMM) equals the fused path."""
    spec = workloads.linear_spec("o_proj", 4096, 4096, workloads.generator(1005), keep_codes=True)
    wrapper = workloads.build_module(spec, "cuda")
    rl = wrapper.rotate_linear
    x = workloads.activations(24, 4096, workloads.generator(1006)).cuda()
    fused = wrapper(x)
    xr = rl.rotation(x.half())                         # the reference's fp16 rotation op
    xq_u, xs_u = torch.ops.paroquant.quant_i8(xr)
    xq_f, xs_f = torch.ops.paroquant.rotate_quant_i8(x, rl.rotation.rot_idx, rl.rotation.rot_cs,
                                                     rl.rotation.scales_f32, rl.rotation.krot, True, True)
    assert_codes_close(to_np(xq_u), to_np(xq_f))
    unfused = MarlinW4A8Linear.forward(rl.qlinear, xr).to(torch.bfloat16)
    assert rel_fro(to_np(unfused), to_np(fused)) < 1e-2
    fp16_chain = rl(x.half())                           # RotateLinearInt4 on fp16 input
    assert fp16_chain.dtype == torch.float16
    assert rel_fro(to_np(fp16_chain), to_np(fused)) < 1e-2


def test_convert_from_wqlinear_checkpoint():
    """WQLinear buffers (pack_intweight layout, scaled_zeros = -s*z) -> convert_model_to_marlin_w4a8."""
    N, K = 1024, 4096
    spec = workloads.linear_spec("k_proj", N, K, workloads.generator(1007), keep_codes=True)
    rl = RotateLinearInt4(K, N, bias=True, dtype=torch.float16, rotation_angles=spec.theta,
                          rotation_pairs=spec.pairs, channel_scales=spec.channel_scales)
    wq = rl.qlinear
    assert isinstance(wq, WQLinear)
    G = K // 128
    wq.qweight.copy_(pack_intweight(spec.w.codes.to(torch.int32)))
    wq.scales.zero_()
    wq.scaled_zeros.zero_()
    wq.scales[:G] = spec.w.awq_scales
    wq.scaled_zeros[:G] = (-(spec.w.awq_scales.float() * spec.w.zeros.float())).half()
    bias = torch.randn(N).half()
    wq.bias.copy_(bias)
    model = torch.nn.Sequential(rl).cuda()
    assert convert_model_to_marlin_w4a8(model) == 1
    assert isinstance(rl.qlinear, MarlinW4A8Linear)
    x = workloads.activations(3, K, workloads.generator(1008))
    y = BF16RotateLinearWrapper(rl)(x.cuda())
    c, s = orot.cos_sin_table(spec.theta.numpy())
    _, q, sx = olin.rotate_quant(to_np(x), spec.pairs.numpy(), c, s, spec.channel_scales.float().reshape(-1).numpy())
    ref = ogemm.w4a8_linear(q, sx, spec.w.codes.numpy(), spec.w.awq_scales.numpy(), spec.w.zeros.numpy(),
                            bias.float().numpy())
    assert_bf16_close(to_np(y), ref)


@pytest.mark.parametrize("M", [1, 16, 96])
def test_graph_capture_replays_match_eager(M):
    """Captured in a HIP graph, every replay (with eager work in between) equals the eager result."""
    spec = workloads.linear_spec("v_proj", 1024, 4096, workloads.generator(1009))
    mod = workloads.build_module(spec, "cuda")
    x = workloads.activations(M, 4096, workloads.generator(1010)).cuda()
    eager = mod(x).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        mod(x)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = mod(x)
    for i in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs"
        _ = mod(x)                        # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5])
@pytest.mark.parametrize("N,K", [(16, 128), (48, 2048), (32, 8192), (1024, 12288), (12288, 4096)])
@pytest.mark.parametrize("krot,flags", [(8, (True, True)), (1, (False, True)), (8, (True, False)), (16, (True, True))])
def test_linear_op_decode_paths(M, N, K, krot, flags):
    """paroquant::w4a8_linear on both of its paths: split rotation + prologue-quantizing GEMM
    (M * K <= 8192, or K >= 8192 and M <= 2), the three-launch split path (K >= 8192 beyond) and row
    rotate+quant + GEMM (otherwise)."""
    print(f"linear op M={M} N={N} K={K} krot={krot} flags={flags}", flush=True)
    g = workloads.generator(zlib.crc32(f"{M}{N}{K}{krot}{flags}".encode()))
    spec = workloads.linear_spec("x", N, K, g, keep_codes=True)
    pairs = torch.cat([spec.pairs] * 2)[:krot]
    theta = torch.cat([spec.theta] * 2)[:krot]
    rot_idx, rot_cs, c, s = packed_rotation(pairs, theta)
    scales = spec.channel_scales.float().reshape(-1)
    wp, wm = torch.ops.paroquant.w4a8_prepack(spec.w.awq_qweight.cuda(), spec.w.awq_scales.cuda(),
                                              spec.w.awq_qzeros.cuda())
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    x = workloads.activations(M, K, g)
    y = torch.ops.paroquant.w4a8_linear(x.cuda(), rot_idx.cuda(), rot_cs.cuda(), scales.cuda(), krot, wp, wm,
                                        bias.cuda(), flags[0], flags[1], torch.bfloat16)
    v = orot.rotate_path_f32(to_np(x), pairs.numpy(), c, s, scales.numpy(), 128, flags[0], flags[1])
    q, sx = oquant.quant_int8_per_token(v)
    ref = ogemm.w4a8_linear(q, sx, spec.w.codes.numpy(), spec.w.awq_scales.numpy(), spec.w.zeros.numpy(),
                            bias.float().numpy())
    assert_bf16_close(to_np(y), ref)


@pytest.mark.parametrize("M", [1, 3, 8])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_linear_op_input_dtypes(M, dtype):
    """fp16 and fp32 activations through paroquant::w4a8_linear, output in the input's dtype."""
    N, K = 64, 4096
    print(f"linear op dtype={dtype} M={M}", flush=True)
    g = workloads.generator(zlib.crc32(f"dt{M}{dtype}".encode()))
    spec = workloads.linear_spec("x", N, K, g, keep_codes=True)
    rot_idx, rot_cs, c, s = packed_rotation(spec.pairs, spec.theta)
    scales = spec.channel_scales.float().reshape(-1)
    wp, wm = torch.ops.paroquant.w4a8_prepack(spec.w.awq_qweight.cuda(), spec.w.awq_scales.cuda(),
                                              spec.w.awq_qzeros.cuda())
    x = workloads.activations(M, K, g).to(dtype)
    y = torch.ops.paroquant.w4a8_linear(x.cuda(), rot_idx.cuda(), rot_cs.cuda(), scales.cuda(), 8, wp, wm, None,
                                        False, True, dtype)
    assert y.dtype == dtype
    v = orot.rotate_path_f32(to_np(x), spec.pairs.numpy(), c, s, scales.numpy(), 128, False, True)
    q, sx = oquant.quant_int8_per_token(v)
    ref = ogemm.w4a8_linear(q, sx, spec.w.codes.numpy(), spec.w.awq_scales.numpy(), spec.w.zeros.numpy(), None)
    assert_bf16_close(to_np(y), ref)


@pytest.mark.parametrize("M", [1, 20])
def test_rows_longer_than_the_fused_kernels(M):
    """K = 16512 (> 16384, the fused kernels' limit) runs rotate -> quant -> GEMM as three ops with the same
    semantics; against the oracle."""
    N, K = 64, 16384 + 128
    spec = workloads.linear_spec("long", N, K, workloads.generator(1300 + M), keep_codes=True)
    mod = workloads.build_module(spec, "cuda")
    x = workloads.activations(M, K, workloads.generator(1400 + M))
    y = mod(x.cuda())
    ref, _, _ = _oracle_linear(spec, to_np(x))
    assert y.shape == (M, N) and y.dtype == torch.bfloat16
    assert_bf16_close(to_np(y), ref)
