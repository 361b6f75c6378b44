"""GPU parity of the W4A16 path (WQLinear.forward, qmodule.py:207-232, and
RotateLinearInt4 over a WQLinear, rotation_linear.py:136-139) against the
oracle (oracle/w4a16.py).

Bar: the kernels form each weight as fp16(q * s + sz) exactly as the oracle
does and accumulate the exact products in float32, so float32 outputs agree
with the float64 oracle to 1e-5 relative (Frobenius) and fp16 / bf16 outputs
to their own rounding (elementwise 2^-10 / 2^-7 relative plus 1e-4 of the
rms).  Against the unrounded weights of the reference's dequant_wqlinear
(paroquant_marlin_w4a8.py:216-224) the outputs stay within 1e-2 relative."""

import functools

import numpy as np
import pytest
import torch

import alpamayo_amd  # noqa: F401
from alpamayo_amd import workloads
from alpamayo_amd.quantization import RotateLinearInt4, WQLinear
from alpamayo_amd.quantization.qmodule import pack_intweight
from oracle import gemm as ogemm
from oracle import rotation as orot
from oracle import w4a16 as ow
from tests.gpu_util import rel_fro, to_np

pytestmark = pytest.mark.gpu

_ULP_REL = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}


def _case(n, k, seed):
    gen = workloads.generator(seed)
    w = workloads.weights(n, k, gen, keep_codes=True)
    s, sz = workloads.w16_scales(w)
    return w, s, sz


@functools.lru_cache(maxsize=None)
def _decode_case(n, k):
    """Weights of one decode shape, their packed form and both oracle weight matrices (float64 [N, K])."""
    w, s, sz = _case(n, k, 3200 + n + k)
    wpack, wmeta = _prepack(w, s, sz)
    codes = w.codes.numpy()
    w16 = ow.dequant_w16(codes, s.numpy(), sz.numpy()).astype(np.float64)
    exact = ogemm.dequant_wqlinear(codes, s.numpy(), sz.numpy())
    return wpack, wmeta, w16, exact


def _prepack(w, s, sz):
    return torch.ops.paroquant.w4a16_prepack(w.awq_qweight.cuda(), s.cuda(), sz.cuda())


def _check(y, ref, out_dtype, exact=None):
    got = to_np(y).astype(np.float64)
    if out_dtype == torch.float32:
        e = rel_fro(got, ref)
        assert e <= 1e-5, f"relative Frobenius error {e:.3e}"
    else:
        e = rel_fro(got, ref)
        assert e <= 2e-3, f"relative Frobenius error {e:.3e}"
        rms = np.sqrt(np.mean(ref ** 2)) + 1e-30
        bad = np.abs(got - ref) > _ULP_REL[out_dtype] * np.abs(ref) + 1e-4 * rms
        assert not bad.any(), f"{bad.sum()} outputs beyond the bound; got {got[bad][:4]} ref {ref[bad][:4]}"
    if exact is not None:
        assert rel_fro(got, exact) <= 1e-2


def test_prepack_layout():
    """Codes as the W4A8 prepack lays them out; metadata s | sz << 16 per (tile, group, column)."""
    n, k = 80, 512
    w, s, sz = _case(n, k, 3101)
    wpack16, wmeta16 = _prepack(w, s, sz)
    wpack8, _ = torch.ops.paroquant.w4a8_prepack(w.awq_qweight.cuda(), w.awq_scales.cuda(), w.awq_qzeros.cuda())
    assert torch.equal(wpack16.cpu(), wpack8.cpu())
    sb = s.view(torch.int16).numpy().astype(np.uint32) & 0xFFFF
    zb = sz.view(torch.int16).numpy().astype(np.uint32) & 0xFFFF
    meta = (sb | (zb << 16)).reshape(k // 128, n // 16, 16).transpose(1, 0, 2)
    got = wmeta16.cpu().numpy().view(np.uint32)
    assert np.array_equal(got, meta)


@pytest.mark.parametrize("n,k", [(256, 256), (4096, 4096), (1024, 4096), (4096, 12288), (12288, 4096)])
@pytest.mark.parametrize("m", [1, 2, 3, 5, 8, 13, 16])
def test_gemm_decode(m, n, k):
    print(f"w4a16 gemm decode m={m} n={n} k={k}", flush=True)
    wpack, wmeta, w16, exact = _decode_case(n, k)
    gen = workloads.generator(3300 + m)
    x = (0.5 * torch.randn(m, k, generator=gen)).to(torch.float16)
    y = torch.ops.paroquant.w4a16_gemm(x.cuda(), wpack, wmeta, None, torch.float16)
    torch.cuda.synchronize()
    xf = x.numpy().astype(np.float64)
    _check(y, xf @ w16.T, torch.float16, exact=xf @ exact.T)


@pytest.mark.parametrize("m,n,k", [(17, 256, 256), (64, 1024, 4096), (100, 272, 384), (300, 1024, 4096),
                                   (300, 16, 128), (1029, 4096, 4096), (3072, 4096, 4096)])
def test_gemm_prefill(m, n, k):
    print(f"w4a16 gemm prefill m={m} n={n} k={k}", flush=True)
    w, s, sz = _case(n, k, 3400 + n + k)
    wpack, wmeta = _prepack(w, s, sz)
    gen = workloads.generator(3500 + m)
    x = (0.5 * torch.randn(m, k, generator=gen)).to(torch.float16)
    y = torch.ops.paroquant.w4a16_gemm(x.cuda(), wpack, wmeta, None, torch.float32)
    torch.cuda.synchronize()
    ref = ow.w4a16_gemm(x.numpy(), w.codes.numpy(), s.numpy(), sz.numpy())
    _check(y, ref, torch.float32)


@pytest.mark.parametrize("m", [3, 40])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bias_dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_gemm_bias_and_output_dtypes(m, out_dtype, bias_dtype):
    n, k = 512, 1024
    w, s, sz = _case(n, k, 3600)
    wpack, wmeta = _prepack(w, s, sz)
    gen = workloads.generator(3601 + m)
    x = torch.randn(m, k, generator=gen).to(torch.float16)
    bias = torch.randn(n, generator=gen).to(bias_dtype)
    y = torch.ops.paroquant.w4a16_gemm(x.cuda(), wpack, wmeta, bias.cuda(), out_dtype)
    torch.cuda.synchronize()
    assert y.dtype == out_dtype and y.shape == (m, n)
    ref = ow.w4a16_gemm(x.numpy(), w.codes.numpy(), s.numpy(), sz.numpy(), to_np(bias))
    _check(y, ref, out_dtype)


@pytest.mark.parametrize("m", [3, 300])
def test_gemm_16bit_outputs_are_rounded_f32(m):
    """bf16 and fp16 outputs equal the float32 output rounded to nearest even by torch, bit for bit (decode and
    prefill kernels): the conversion is the last step."""
    n, k = 512, 1024
    w, s, sz = _case(n, k, 3700)
    wpack, wmeta = _prepack(w, s, sz)
    gen = workloads.generator(3701 + m)
    x = torch.randn(m, k, generator=gen).to(torch.float16).cuda()
    bias = torch.randn(n, generator=gen).to(torch.float16).cuda()
    y32 = torch.ops.paroquant.w4a16_gemm(x, wpack, wmeta, bias, torch.float32)
    for dt in (torch.bfloat16, torch.float16):
        y = torch.ops.paroquant.w4a16_gemm(x, wpack, wmeta, bias, dt)
        assert torch.equal(y.view(torch.int16), y32.to(dt).view(torch.int16)), dt


def test_gemm_empty_and_leading_dims():
    n, k = 256, 512
    w, s, sz = _case(n, k, 3700)
    wpack, wmeta = _prepack(w, s, sz)
    y0 = torch.ops.paroquant.w4a16_gemm(torch.empty(0, k, dtype=torch.float16, device="cuda"), wpack, wmeta, None,
                                        torch.float16)
    assert y0.shape == (0, n)
    x = torch.randn(2, 3, k, generator=workloads.generator(3701)).to(torch.float16)
    y = torch.ops.paroquant.w4a16_gemm(x.cuda(), wpack, wmeta, None, torch.float32)
    assert y.shape == (2, 3, n)
    ref = ow.w4a16_gemm(x.reshape(6, k).numpy(), w.codes.numpy(), s.numpy(), sz.numpy())
    _check(y.reshape(6, n), ref, torch.float32)
    with pytest.raises(RuntimeError, match="float16"):
        torch.ops.paroquant.w4a16_gemm(x.cuda().float(), wpack, wmeta, None, torch.float32)


@pytest.mark.parametrize("m", [1, 4, 16, 17, 300])
@pytest.mark.parametrize("x_dtype,input_fp16", [(torch.float16, False), (torch.bfloat16, True),
                                                (torch.float32, False)])
def test_linear_rotation_then_gemm(m, x_dtype, input_fp16):
    print(f"w4a16 linear m={m} x={x_dtype} input_fp16={input_fp16}", flush=True)
    spec = workloads.linear_spec("o_proj", 1024, 4096, workloads.generator(3800), keep_codes=True)
    x = workloads.activations(m, 4096, workloads.generator(3801 + m)).to(x_dtype)
    from tests.gpu_util import packed_rotation

    rot_idx, rot_cs, c, sn = packed_rotation(spec.pairs, spec.theta)
    s, sz = workloads.w16_scales(spec.w)
    wpack, wmeta = _prepack(spec.w, s, sz)
    scales = spec.channel_scales.float().reshape(-1)
    y = torch.ops.paroquant.w4a16_linear(x.cuda(), rot_idx.cuda(), rot_cs.cuda(), scales.cuda(), 8, wpack, wmeta,
                                         None, input_fp16, torch.float32)
    torch.cuda.synchronize()
    ref, _ = ow.rotate_linear_w16(to_np(x).astype(np.float32), spec.pairs.numpy(), c, sn, scales.numpy(),
                                  spec.w.codes.numpy(), s.numpy(), sz.numpy(), input_fp16=input_fp16)
    # a rotated value may land one fp16 ulp away from the oracle's (fp32 rounding order of the
    # Givens chain), so the bar here is the rounding of A, not the accumulation
    e = rel_fro(to_np(y), ref)
    assert e <= 1e-3, f"relative Frobenius error {e:.3e}"


def _wq_module(spec, bias=None):
    q = WQLinear(4, 128, spec.K, spec.N, bias is not None, dtype=torch.float16)
    G = spec.K // 128
    s, sz = workloads.w16_scales(spec.w)
    q.qweight.copy_(pack_intweight(spec.w.codes.to(torch.int32)))
    q.scales[:G].copy_(s)
    q.scaled_zeros[:G].copy_(sz)
    if bias is not None:
        q.bias.copy_(bias)
    return q.cuda(), s, sz


@pytest.mark.parametrize("m", [1, 7, 8, 64])
def test_wqlinear_forward(m):
    spec = workloads.linear_spec("k_proj", 1024, 4096, workloads.generator(3900), keep_codes=True)
    bias = torch.randn(1024, generator=workloads.generator(3901)).to(torch.float16)
    q, s, sz = _wq_module(spec, bias)
    keys = set(q.state_dict().keys())
    assert keys == {"qweight", "scales", "scaled_zeros", "bias"}
    x = torch.randn(m, 4096, generator=workloads.generator(3902 + m)).to(torch.float16)
    y = q(x.cuda())
    torch.cuda.synchronize()
    assert y.dtype == torch.float16 and q.prepared
    ref = ow.w4a16_gemm(x.numpy(), spec.w.codes.numpy(), s.numpy(), sz.numpy(), bias.numpy())
    _check(y, ref, torch.float16)


def test_wqlinear_reprepares_after_buffer_update():
    spec = workloads.linear_spec("k_proj", 256, 512, workloads.generator(3950), keep_codes=True)
    q, s, sz = _wq_module(spec)
    x = torch.randn(4, 512, generator=workloads.generator(3951)).to(torch.float16).cuda()
    y1 = q(x).clone()
    spec2 = workloads.linear_spec("k_proj", 256, 512, workloads.generator(3952), keep_codes=True)
    q.qweight.copy_(pack_intweight(spec2.w.codes.to(torch.int32)).cuda())   # e.g. load_state_dict
    assert not q.prepared
    y2 = q(x)
    torch.cuda.synchronize()
    ref2 = ow.w4a16_gemm(to_np(x), spec2.w.codes.numpy(), s.numpy(), sz.numpy())
    _check(y2, ref2, torch.float16)
    assert not torch.equal(y1, y2)


@pytest.mark.parametrize("m", [1, 16, 100])
def test_rotate_linear_int4_with_wqlinear(m):
    spec = workloads.linear_spec("gate_proj", 2048, 1024, workloads.generator(4000), keep_codes=True)
    rl = workloads.build_w16_module(spec, "cuda")
    assert isinstance(rl, RotateLinearInt4) and isinstance(rl.qlinear, WQLinear)
    x = workloads.activations(m, 1024, workloads.generator(4001 + m)).to(torch.float16)
    y = rl(x.cuda())
    torch.cuda.synchronize()
    assert y.dtype == torch.float16
    c, sn = orot.cos_sin_table(spec.theta.numpy())
    s, sz = workloads.w16_scales(spec.w)
    ref, _ = ow.rotate_linear_w16(x.float().numpy(), spec.pairs.numpy(), c, sn,
                                  spec.channel_scales.float().reshape(-1).numpy(), spec.w.codes.numpy(), s.numpy(),
                                  sz.numpy())
    assert rel_fro(to_np(y), ref) <= 2e-3


@pytest.mark.parametrize("m", [1, 200])
def test_graph_replay(m):
    spec = workloads.linear_spec("o_proj", 1024, 2048, workloads.generator(4100), keep_codes=True)
    rl = workloads.build_w16_module(spec, "cuda")
    x = workloads.activations(m, 2048, workloads.generator(4101 + m)).to(torch.float16).cuda()
    eager = rl(x).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        rl(x)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = rl(x)
    for i in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        rl(x + 1.0)   # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("m", [1, 5, 16, 20])
@pytest.mark.parametrize("ns", [(1024, 1040, 64), (12288, 12288), (4096, 1024, 1024)])
def test_linear_group_matches_single_linears(m, ns):
    """paroquant::w4a16_linear_group (one rotation launch; one GEMM launch at m <= 16, tiles of every member
    in one grid) gives each member what paroquant::w4a16_linear gives it alone.  The group's launch may split
    K over a different number of waves (its workgroup count is the members' total), which changes the
    float32 summation order: the outputs then agree to one rounding of the output format."""
    print(f"w4a16 group m={m} ns={ns}", flush=True)
    from tests.gpu_util import packed_rotation

    k = 4096
    x = workloads.activations(m, k, workloads.generator(3900 + m)).cuda()
    args = []
    for i, n in enumerate(ns):
        spec = workloads.linear_spec(f"m{i}", n, k, workloads.generator(3910 + 7 * i + n), keep_codes=True)
        rot_idx, rot_cs, _, _ = packed_rotation(spec.pairs, spec.theta)
        s, sz = workloads.w16_scales(spec.w)
        wpack, wmeta = _prepack(spec.w, s, sz)
        scales = spec.channel_scales.float().reshape(-1).cuda()
        bias = (torch.randn(n, generator=torch.Generator().manual_seed(i)) * 0.1).half().cuda() if i == 0 else None
        args.append((rot_idx.cuda(), rot_cs.cuda(), scales, wpack, wmeta, bias))
    outs = torch.ops.paroquant.w4a16_linear_group(x, [a[0] for a in args], [a[1] for a in args],
                                                  [a[2] for a in args], 8, [a[3] for a in args],
                                                  [a[4] for a in args], [a[5] for a in args], True,
                                                  torch.bfloat16)
    for (ri, rc, sc, wp, wm, b), y, n in zip(args, outs, ns):
        ref = torch.ops.paroquant.w4a16_linear(x, ri, rc, sc, 8, wp, wm, b, True, torch.bfloat16)
        torch.cuda.synchronize()
        assert y.shape == (m, n)
        yf, rf = y.float(), ref.float()
        rms = rf.pow(2).mean().sqrt()
        assert torch.all((yf - rf).abs() <= _ULP_REL[torch.bfloat16] * rf.abs() + 1e-4 * rms)


@pytest.mark.parametrize("m", [1, 3])
@pytest.mark.parametrize("k", [384, 1152])
def test_linear_group_member_blocks_aligned_small_k(m, k):
    """Groups whose per-member scratch (fp16 rows + group maxima) is not a multiple of 16 bytes before
    rounding (m * (k / 128) not a multiple of 4): every member's rows still start 256-byte aligned, and each
    member gets what paroquant::w4a16_linear gives it alone."""
    print(f"w4a16 group small k={k} m={m}", flush=True)
    from tests.gpu_util import packed_rotation

    ns = (64, 48, 32)
    x = workloads.activations(m, k, workloads.generator(3950 + m + k)).cuda()
    args = []
    for i, n in enumerate(ns):
        spec = workloads.linear_spec(f"s{i}", n, k, workloads.generator(3960 + 7 * i + n + k), keep_codes=True)
        rot_idx, rot_cs, _, _ = packed_rotation(spec.pairs, spec.theta)
        s, sz = workloads.w16_scales(spec.w)
        wpack, wmeta = _prepack(spec.w, s, sz)
        args.append((rot_idx.cuda(), rot_cs.cuda(), spec.channel_scales.float().reshape(-1).cuda(), wpack, wmeta))
    need = alpamayo_amd.ops._lib.load().pq_w4a16_linear_group_workspace_size(m, k, len(ns))
    assert need % (256 * len(ns)) == 0
    outs = torch.ops.paroquant.w4a16_linear_group(x, [a[0] for a in args], [a[1] for a in args],
                                                  [a[2] for a in args], 8, [a[3] for a in args],
                                                  [a[4] for a in args], [None] * len(ns), True, torch.bfloat16)
    for (ri, rc, sc, wp, wm), y, n in zip(args, outs, ns):
        ref = torch.ops.paroquant.w4a16_linear(x, ri, rc, sc, 8, wp, wm, None, True, torch.bfloat16)
        torch.cuda.synchronize()
        assert y.shape == (m, n)
        yf, rf = y.float(), ref.float()
        rms = rf.pow(2).mean().sqrt()
        assert torch.all((yf - rf).abs() <= _ULP_REL[torch.bfloat16] * rf.abs() + 1e-4 * rms)
