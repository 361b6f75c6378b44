"""A shared-input group behind a decoder layer's residual add or its gated-MLP
activation (paroquant::w4a8_linear_group_fused, PQ_PRO_ADD / PQ_PRO_SWIGLU):
the rows the rotation reads -- s = x + residual, act = silu(gate) * up --
against torch's own ops and the oracle, and the members' outputs against the
plain group run on those rows (bit-identical: same rotation input) and against
the oracle chain.  The RMSNorm prologue is covered by test_gpu_rmsnorm.py."""

import zlib

import numpy as np
import pytest
import torch

import alpamayo_amd  # noqa: F401
from alpamayo_amd import _lib, workloads
from oracle import linear as olin
from oracle import rmsnorm as orms
from tests.gpu_util import assert_bf16_close, to_np
from tests.test_gpu_group import _members, _oracle

pytestmark = pytest.mark.gpu

CASES = [
    # (M, K, member Ns): the split pair (M*K <= 8192, or M <= 2 for K >= 8192), the three-launch
    # path (K >= 4096 up to 64 tokens), the row rotate+quant path (short rows at a few tokens, and
    # from 65 tokens), ragged row counts
    (1, 4096, (4096, 1024, 1024)),
    (1, 12288, (4096,)),
    (3, 12288, (4096,)),
    (7, 12288, (1024, 48)),
    (3, 4096, (1024, 1024)),
    (16, 12288, (4096,)),
    (17, 12288, (4096,)),
    (24, 12288, (1024, 48)),
    (32, 16384, (4096,)),
    (48, 4096, (4096, 1024, 1024)),
    (64, 12288, (4096,)),
    (65, 4096, (1024, 64)),
    (300, 4096, (4096, 1024)),
    (1029, 2048, (1040, 16)),
    (6, 2048, (1024, 64)),
    (2053, 512, (1040, 16)),   # from 2048 rows: blocks sized to fill rounds (three rows here) and a remainder
]


def _args(mbs, krot, flags):
    return ([m["rot_idx"] for m in mbs], [m["rot_cs"] for m in mbs], [m["scales"] for m in mbs], krot,
            [m["wp"] for m in mbs], [m["wm"] for m in mbs], [m["bias"] for m in mbs], flags[0], flags[1],
            torch.bfloat16)


@pytest.mark.parametrize("M,K,ns", CASES)
def test_residual_add_group(M, K, ns):
    print(f"add group M={M} K={K} ns={ns}", flush=True)
    seed = zlib.crc32(f"add{M}-{K}-{ns}".encode())
    krot, flags = 8, (True, True)
    mbs = _members(ns, K, krot, seed, with_bias=True)
    g = workloads.generator(seed + 1)
    x, r = workloads.activations(M, K, g).cuda(), workloads.activations(M, K, g).cuda()
    args = _args(mbs, krot, flags)
    outs = torch.ops.paroquant.w4a8_linear_group_fused(x, r, None, 0.0, _lib.PQ_PRO_ADD, *args, False, True)
    assert len(outs) == len(ns) + 1
    s = outs[-1]
    assert torch.equal(s, x + r), "the sum is torch's bf16 add"
    plain = torch.ops.paroquant.w4a8_linear_group(x + r, *args)
    s_np = to_np(s)
    for mb, y, yp, N in zip(mbs, outs[:len(ns)], plain, ns):
        assert y.shape == (M, N)
        assert torch.equal(y, yp), "the fused add must feed the rotation exactly the sum it writes"
        assert_bf16_close(to_np(y), _oracle(mb, s_np, flags))


@pytest.mark.parametrize("M,K,ns", CASES)
def test_swiglu_group(M, K, ns):
    print(f"swiglu group M={M} K={K} ns={ns}", flush=True)
    seed = zlib.crc32(f"glu{M}-{K}-{ns}".encode())
    krot, flags = 8, (True, True)
    mbs = _members(ns, K, krot, seed, with_bias=True)
    g = workloads.generator(seed + 1)
    gate, up = workloads.activations(M, K, g).cuda(), workloads.activations(M, K, g).cuda()
    args = _args(mbs, krot, flags)
    outs = torch.ops.paroquant.w4a8_linear_group_fused(gate, up, None, 0.0, _lib.PQ_PRO_SWIGLU, *args, True, False)
    assert len(outs) == len(ns) + 1
    act = outs[-1]
    ref_t = torch.nn.functional.silu(gate) * up          # torch's ops on the GPU, bf16 module rounding
    a, b = olin.bf16_bits(to_np(act)).astype(np.int32), olin.bf16_bits(to_np(ref_t)).astype(np.int32)
    assert np.abs(a - b).max(initial=0) <= 1 and np.mean(a == b) >= 0.999
    ref_o = orms.swiglu(to_np(gate), to_np(up), "bf16")
    o = olin.bf16_bits(ref_o).astype(np.int32)
    assert np.abs(a - o).max(initial=0) <= 2 and np.mean(a == o) >= 0.999
    plain = torch.ops.paroquant.w4a8_linear_group(act, *args)
    for mb, y, yp, N in zip(mbs, outs[:len(ns)], plain, ns):
        assert y.shape == (M, N)
        assert torch.equal(y, yp), "the fused activation must feed the rotation exactly the rows it writes"
        assert_bf16_close(to_np(y), _oracle(mb, ref_o, flags))


@pytest.mark.parametrize("M", [1, 16])
def test_module_options_and_graph_replay(M):
    """SharedInputRotateLinears(x, residual=r) and .forward_swiglu(gate, up) inside a captured graph: fused
    into the rotation at M = 1 (split path), separate torch ops at M = 16 (row path)."""
    K = 4096
    g = workloads.generator(4343)
    from alpamayo_amd.quantization import SharedInputRotateLinears
    qkv = SharedInputRotateLinears([workloads.build_module(workloads.linear_spec(n, N, K, g), "cuda")
                                    for n, N in (("q", 1024), ("k", 512))])
    down = SharedInputRotateLinears([workloads.build_module(workloads.linear_spec("down", 1024, K, g), "cuda")])
    x, r, gt, up = (workloads.activations(M, K, g).cuda() for _ in range(4))

    def step():
        q, k, s = qkv(x, residual=r, return_sum=True)
        (d, act) = down.forward_swiglu(gt, up, return_act=True)
        return q, k, s, d, act

    eager = [t.clone() for t in step()]
    assert torch.equal(eager[2], x + r)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        step()
    torch.cuda.current_stream().wait_stream(st)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        cap = step()
    for _ in range(3):
        torch.cuda.synchronize()
        junk = torch.randn(1 << 20, device="cuda").sum()   # eager work between replays
        gr.replay()
        torch.cuda.synchronize()
        for a, b in zip(eager, cap):
            assert torch.equal(a, b)
        del junk
    with pytest.raises(ValueError):
        qkv(x, residual=r, return_normed=True)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("M,K", [(1, 4096), (16, 4096), (300, 4096), (1, 12288), (16, 12288)])
def test_prologues_other_dtypes(dtype, M, K):
    """The residual add and the SwiGLU prologue on fp16 and float32 activations,
    on the split pair, the three-launch path and the row kernel: the sum equal
    to torch's add in that dtype, the activation within one ulp of torch's
    silu(gate) * up in fp16 (float32: rtol 1e-5, the exponentials may differ
    in their last bits) and within two of the oracle's, and the members'
    outputs equal to the plain group run on the rows the kernel wrote."""
    print(f"prologues dtype={dtype} M={M} K={K}", flush=True)
    seed = zlib.crc32(f"pro-dt-{dtype}-{M}-{K}".encode())
    krot, flags = 8, (True, True)
    mbs = _members((1024, 48), K, krot, seed, with_bias=True)
    g = workloads.generator(seed + 1)
    x, r = (workloads.activations(M, K, g).to(dtype).cuda() for _ in range(2))
    args = _args(mbs, krot, flags)
    outs = torch.ops.paroquant.w4a8_linear_group_fused(x, r, None, 0.0, _lib.PQ_PRO_ADD, *args, False, True)
    s = outs[-1]
    assert s.dtype == dtype and torch.equal(s, x + r)
    for y, yp in zip(outs[:2], torch.ops.paroquant.w4a8_linear_group(x + r, *args)):
        assert torch.equal(y, yp)
    outs = torch.ops.paroquant.w4a8_linear_group_fused(x, r, None, 0.0, _lib.PQ_PRO_SWIGLU, *args, True, False)
    act = outs[-1]
    ref_t = torch.nn.functional.silu(x) * r
    if dtype == torch.float16:
        a = act.cpu().view(torch.int16).numpy().astype(np.int32)
        b = ref_t.cpu().view(torch.int16).numpy().astype(np.int32)
        assert np.abs(a - b).max(initial=0) <= 1 and np.mean(a == b) >= 0.999
        ref_o = orms.swiglu(to_np(x), to_np(r), "f16").astype(np.float16)
        o = torch.from_numpy(ref_o).view(torch.int16).numpy().astype(np.int32)
        assert np.abs(a - o).max(initial=0) <= 2 and np.mean(a == o) >= 0.999
    else:
        np.testing.assert_allclose(to_np(act), to_np(ref_t), rtol=1e-5, atol=1e-30)
        np.testing.assert_allclose(to_np(act), orms.swiglu(to_np(x), to_np(r), "f32"), rtol=1e-5, atol=1e-30)
    for y, yp in zip(outs[:2], torch.ops.paroquant.w4a8_linear_group(act, *args)):
        assert torch.equal(y, yp)
