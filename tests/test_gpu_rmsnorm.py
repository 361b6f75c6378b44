"""A shared-input group behind the decoder layer's RMSNorm
(paroquant::w4a8_linear_group_rmsnorm): the normalized rows h and the residual
sum s against the RMSNorm oracle (Qwen3VLTextRMSNorm.forward,
modeling_qwen3_vl.py:354-359), and the members' outputs against the plain
group run on the h the kernel wrote (bit-identical: same rotation input) and
against the oracle chain fed that h.  (h may differ from the oracle's by one
bf16 ulp in up to 0.1 % of its elements -- the float32 rsqrt -- and such a
difference can move an int8 code by one, so the chain is checked stage by
stage.)"""

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
    # path (K >= 4096 up to 32 tokens), the row rotate+quant path (short rows at a few tokens, and
    # from 33 tokens), ragged row counts
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
