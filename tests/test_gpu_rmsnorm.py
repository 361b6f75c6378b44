"""A shared-input group behind the decoder layer's RMSNorm
(paroquant::w4a8_linear_group_rmsnorm): the normalized rows h and the residual
sum s against the RMSNorm oracle (Qwen3VLTextRMSNorm.forward,
modeling_qwen3_vl.py:354-359), and the members' outputs against the plain
group run on the h the kernel wrote (bit-identical: same rotation input) and
against the oracle chain fed that h.  (h may differ from the oracle's by one
bf16 ulp in up to 0.1 % of its elements -- the float32 rsqrt -- and such a
difference can move an int8 code by one, so the chain is checked stage by
stage.)  Each row of h is also checked to be exactly the oracle's formula for
an r within a few float32 ulps of the oracle's."""

import zlib

import numpy as np
import pytest
import torch

import alpamayo_amd  # noqa: F401
from alpamayo_amd import workloads
from oracle import linear as olin
from oracle import rmsnorm as orms
from tests.gpu_util import assert_bf16_close, to_np
from tests.test_gpu_group import _members, _oracle

pytestmark = pytest.mark.gpu


def _bits_close(got_np, ref_np, min_equal=0.999):
    g = olin.bf16_bits(got_np).astype(np.int32)
    r = olin.bf16_bits(ref_np).astype(np.int32)
    assert np.abs(g - r).max(initial=0) <= 1
    assert np.mean(g == r) >= min_equal


CASES = [
    # (M, K, member Ns): the split pair (M*K <= 8192, or M <= 2 for K >= 8192), the three-launch
    # path (K >= 4096 up to 64 tokens), the row rotate+quant path (short rows at a few tokens, and
    # from 65 tokens), ragged row counts
    (1, 4096, (4096, 1024, 1024)),
    (3, 4096, (1024, 1024)),
    (1, 12288, (4096,)),
    (4, 8192, (1024,)),
    (13, 8192, (1024, 64)),
    (2, 2048, (1024, 64)),
    (16, 4096, (1024, 512)),
    (17, 12288, (4096,)),
    (24, 12288, (1024, 48)),
    (32, 16384, (4096,)),
    (48, 4096, (4096, 1024, 1024)),
    (64, 12288, (4096,)),
    (65, 4096, (1024, 64)),
    (300, 4096, (4096, 1024, 1024)),
    (1029, 2048, (1040, 16)),
    (6, 2048, (1024, 64)),
    (2053, 512, (1040, 16)),   # from 2048 rows: blocks sized to fill rounds (three rows here) and a remainder
]


@pytest.mark.parametrize("M,K,ns", CASES)
@pytest.mark.parametrize("with_res", [True, False])
def test_rmsnorm_group(M, K, ns, with_res):
    print(f"rmsnorm group M={M} K={K} ns={ns} res={with_res}", flush=True)
    seed = zlib.crc32(f"rms{M}-{K}-{ns}-{with_res}".encode())
    krot, flags = 8, (True, True)
    mbs = _members(ns, K, krot, seed, with_bias=True)
    g = workloads.generator(seed + 1)
    x = workloads.activations(M, K, g)
    res = workloads.activations(M, K, g) if with_res else None
    w = (0.8 + 0.4 * torch.rand(K, generator=g)).to(torch.bfloat16)
    args = ([m["rot_idx"] for m in mbs], [m["rot_cs"] for m in mbs], [m["scales"] for m in mbs], krot,
            [m["wp"] for m in mbs], [m["wm"] for m in mbs], [m["bias"] for m in mbs], flags[0], flags[1],
            torch.bfloat16)
    outs = torch.ops.paroquant.w4a8_linear_group_rmsnorm(x.cuda(), res.cuda() if with_res else None, w.cuda(), 1e-6,
                                                         *args, True, with_res)
    assert len(outs) == len(ns) + 1 + int(with_res)
    h_gpu = outs[len(ns)]
    h_ref, s_ref = orms.rmsnorm(to_np(x), to_np(w), 1e-6, to_np(res) if with_res else None, "bf16")
    _bits_close(to_np(h_gpu), h_ref)
    assert _rows_match_some_r(to_np(h_gpu), to_np(x), to_np(res) if with_res else None, to_np(w), 1e-6, "bf16")
    if with_res:
        np.testing.assert_array_equal(olin.bf16_bits(to_np(outs[-1])), olin.bf16_bits(s_ref))
    plain = torch.ops.paroquant.w4a8_linear_group(h_gpu, *args)
    for mb, y, yp, N in zip(mbs, outs[:len(ns)], plain, ns):
        assert y.shape == (M, N)
        assert torch.equal(y, yp), "the fused norm must feed the rotation exactly the h it writes"
        assert_bf16_close(to_np(y), _oracle(mb, to_np(h_gpu), flags))


@pytest.mark.parametrize("K", [4096, 4224])
def test_same_bits_on_every_path(K):
    """The normalized rows do not depend on the path: the row kernel (one wave
    sums each row), the split pair at M = 2 (one wave, all of a row's chunk
    classes) and the split rotations with one row per wave at M = 1 and
    M = 16 (the waves of a workgroup each sum some classes and share them)
    give the same bits for the same rows.  K = 4224 leaves 33 groups (a
    workgroup with idle waves) and rows whose lanes hold unequal chunk counts."""
    print(f"rmsnorm same bits K={K}", flush=True)
    seed = zlib.crc32(f"rms-paths-{K}".encode())
    krot, flags = 8, (True, True)
    mbs = _members((1024,), K, krot, seed, with_bias=False)
    g = workloads.generator(seed + 1)
    x = workloads.activations(300, K, g).cuda()
    res = workloads.activations(300, K, g).cuda()
    w = (0.8 + 0.4 * torch.rand(K, generator=g)).to(torch.bfloat16).cuda()
    args = ([m["rot_idx"] for m in mbs], [m["rot_cs"] for m in mbs], [m["scales"] for m in mbs], krot,
            [m["wp"] for m in mbs], [m["wm"] for m in mbs], [m["bias"] for m in mbs], flags[0], flags[1],
            torch.bfloat16)

    def normed(m):
        outs = torch.ops.paroquant.w4a8_linear_group_rmsnorm(x[:m], res[:m], w, 1e-6, *args, True, False)
        return outs[1]

    full = normed(300)
    for m in (16, 2, 1):
        assert torch.equal(normed(m), full[:m]), f"M={m}"
    h_ref, _ = orms.rmsnorm(to_np(x), to_np(w), 1e-6, to_np(res), "bf16")
    _bits_close(to_np(full), h_ref)


def _rows_match_some_r(h_gpu, x, res, w, eps, tag, span=128):
    """Whether each row of h_gpu is exactly the oracle's h = round(w * round(s * r'))
    for one r' within `span` float32 ulps of the oracle's r (the float32 sum
    of squares in the kernel's association and the oracle's float64 sum give
    r's that differ in their last bits; any other difference fails)."""
    s = orms.residual_sum(x, res, tag)
    r = orms.rms_factor(s, eps)
    w = np.asarray(w, dtype=np.float32)
    ok = np.zeros(h_gpu.shape[0], dtype=bool)
    for d in range(-span, span + 1):
        rr = (r.view(np.int32) + np.int32(d)).view(np.float32)
        h = orms.round_to(w * orms.round_to(s * rr, tag), tag)
        ok |= np.all(h == h_gpu, axis=-1)
        if ok.all():
            return True
    return bool(ok.all())


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("M", [1, 2, 16, 300])
def test_rmsnorm_other_dtypes(dtype, M):
    """fp16 and float32 activations through the fused RMSNorm on each path
    (M = 1 and 16: split rotations sharing the row sum across waves; M = 2:
    one wave sums the row; M = 300: the row kernel): h against the oracle
    (each row exactly the oracle's formula for an r within a few float32
    ulps of the oracle's: the sums of squares differ in their last bits; an
    fp16 h can then move by two ulps, h = round(w * round(s * r)) with w up
    to 1.2), the residual sum exact, the members' outputs equal to the plain
    group run on the h the kernel wrote, and every path's h equal to the row
    kernel's."""
    print(f"rmsnorm dtype={dtype} M={M}", flush=True)
    K = 4096
    seed = zlib.crc32(f"rms-dt-{dtype}-{M}".encode())
    krot, flags = 8, (True, True)
    mbs = _members((1024, 64), K, krot, seed, with_bias=True)
    g = workloads.generator(seed + 1)
    x = workloads.activations(300, K, g).to(dtype).cuda()
    res = workloads.activations(300, K, g).to(dtype).cuda()
    w = (0.8 + 0.4 * torch.rand(K, generator=g)).to(dtype).cuda()
    args = ([m["rot_idx"] for m in mbs], [m["rot_cs"] for m in mbs], [m["scales"] for m in mbs], krot,
            [m["wp"] for m in mbs], [m["wm"] for m in mbs], [m["bias"] for m in mbs], flags[0], flags[1],
            torch.bfloat16)
    outs = torch.ops.paroquant.w4a8_linear_group_rmsnorm(x[:M], res[:M], w, 1e-6, *args, True, True)
    h_gpu, s_gpu = outs[2], outs[3]
    assert h_gpu.dtype == dtype and s_gpu.dtype == dtype
    tag = "f16" if dtype == torch.float16 else "f32"
    h_ref, s_ref = orms.rmsnorm(to_np(x[:M]), to_np(w), 1e-6, to_np(res[:M]), tag)
    np.testing.assert_array_equal(to_np(s_gpu), s_ref)
    hg = to_np(h_gpu).astype(np.float32)
    if dtype == torch.float16:   # (float32: a last-bit change of r reaches most elements)
        assert np.mean(hg == h_ref) >= 0.995
    assert _rows_match_some_r(hg, to_np(x[:M]), to_np(res[:M]), to_np(w), 1e-6, tag)
    plain = torch.ops.paroquant.w4a8_linear_group(h_gpu, *args)
    for y, yp in zip(outs[:2], plain):
        assert torch.equal(y, yp), "the fused norm must feed the rotation exactly the h it writes"
    if M < 300:
        full = torch.ops.paroquant.w4a8_linear_group_rmsnorm(x, res, w, 1e-6, *args, True, False)[2]
        assert torch.equal(h_gpu, full[:M])


@pytest.mark.parametrize("krot,flags", [(16, (True, True)), (1, (False, False)), (8, (True, False))])
@pytest.mark.parametrize("M", [1, 16, 300])
def test_rmsnorm_other_rotations(krot, flags, M):
    """The fused RMSNorm with 16 and 1 Givens layers and with the other input /
    row-buffer flags (no fp16 input cast, float32 rotated rows), on the split
    rotation sharing the row sum (M = 1, 16) and the row kernel (M = 300)."""
    print(f"rmsnorm krot={krot} flags={flags} M={M}", flush=True)
    K = 4096
    seed = zlib.crc32(f"rms-rot-{krot}-{flags}-{M}".encode())
    mbs = _members((1024, 64), K, krot, seed, with_bias=True)
    g = workloads.generator(seed + 1)
    x, res = (workloads.activations(M, K, g) for _ in range(2))
    w = (0.8 + 0.4 * torch.rand(K, generator=g)).to(torch.bfloat16)
    args = ([m["rot_idx"] for m in mbs], [m["rot_cs"] for m in mbs], [m["scales"] for m in mbs], krot,
            [m["wp"] for m in mbs], [m["wm"] for m in mbs], [m["bias"] for m in mbs], flags[0], flags[1],
            torch.bfloat16)
    outs = torch.ops.paroquant.w4a8_linear_group_rmsnorm(x.cuda(), res.cuda(), w.cuda(), 1e-6, *args, True, True)
    h_gpu = outs[2]
    assert _rows_match_some_r(to_np(h_gpu), to_np(x), to_np(res), to_np(w), 1e-6, "bf16")
    plain = torch.ops.paroquant.w4a8_linear_group(h_gpu, *args)
    for mb, y, yp in zip(mbs, outs[:2], plain):
        assert torch.equal(y, yp), "the fused norm must feed the rotation exactly the h it writes"
        assert_bf16_close(to_np(y), _oracle(mb, to_np(h_gpu), flags))


def test_module_option_and_graph_replay():
    """SharedInputRotateLinears(norm_weight=...) inside a captured graph, replayed with eager work between."""
    K = 4096
    g = workloads.generator(4242)
    mods = [workloads.build_module(workloads.linear_spec(n, N, K, g), "cuda")
            for n, N in (("gate", 1024), ("up", 1024))]
    from alpamayo_amd.quantization import SharedInputRotateLinears
    grp = SharedInputRotateLinears(mods)
    w = (0.8 + 0.4 * torch.rand(K, generator=g)).to(torch.bfloat16).cuda()
    x = workloads.activations(1, K, g).cuda()
    r = workloads.activations(1, K, g).cuda()
    eager = grp(x, norm_weight=w, eps=1e-6, residual=r, return_normed=True, return_sum=True)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        grp(x, norm_weight=w, eps=1e-6, residual=r, return_normed=True, return_sum=True)
    torch.cuda.current_stream().wait_stream(s)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        cap = grp(x, norm_weight=w, eps=1e-6, residual=r, return_normed=True, return_sum=True)
    for _ in range(3):
        torch.cuda.synchronize()
        junk = torch.randn(1 << 20, device="cuda").sum()   # eager work between replays
        gr.replay()
        torch.cuda.synchronize()
        for a, b in zip(eager, cap):
            assert torch.equal(a, b)
        del junk
    assert torch.equal(eager[3], (x + r))
    with pytest.raises(ValueError):
        grp(x, residual=r, return_normed=True)   # the add alone has no normalized rows
