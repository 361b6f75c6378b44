"""The grouped W4A8 linear in two calls (pq_w4a8_linear_group_stage: the rotation / quant launches, then the
GEMM launch) against the one-call form (paroquant::w4a8_linear_group / _fused): bit-identical outputs on every
path (split pair, long rows, row kernel with the decode and the prefill GEMM), with a prologue, and when each
stage is captured in a graph of its own and replayed."""

import zlib

import pytest
import torch

import alpamayo_amd  # noqa: F401
from alpamayo_amd import _lib, ops, workloads
from tests.test_gpu_group import _members

pytestmark = pytest.mark.gpu

CASES = [(1, 4096, (4096, 1024, 1024)), (2, 12288, (4096,)), (5, 12288, (1024, 48)), (16, 4096, (1024, 512)),
         (24, 4096, (4096,)), (300, 4096, (4096, 1024)), (3072, 4096, (4096, 1024, 1024))]


def _lists(mbs):
    return ([m["rot_idx"] for m in mbs], [m["rot_cs"] for m in mbs], [m["scales"] for m in mbs], 8,
            [m["wp"] for m in mbs], [m["wm"] for m in mbs], [m["bias"] for m in mbs])


@pytest.mark.parametrize("M,K,ns", CASES)
def test_two_stages_equal_one_call(M, K, ns):
    print(f"stages M={M} K={K} ns={ns}", flush=True)
    seed = zlib.crc32(f"stg{M}-{K}-{ns}".encode())
    mbs = _members(ns, K, 8, seed, with_bias=True)
    x = workloads.activations(M, K, workloads.generator(seed + 1)).cuda()
    ref = torch.ops.paroquant.w4a8_linear_group(x, *_lists(mbs), True, True, torch.bfloat16)
    st = ops.W4A8GroupStages(x, *_lists(mbs))
    st.rotate()
    outs = st.gemm()
    for y, r in zip(outs, ref):
        assert torch.equal(y, r)


@pytest.mark.parametrize("M,K,ns", [(1, 4096, (4096, 1024, 1024)), (16, 4096, (1024,)), (300, 4096, (1024,))])
def test_two_stages_with_rmsnorm(M, K, ns):
    seed = zlib.crc32(f"stgr{M}-{K}".encode())
    mbs = _members(ns, K, 8, seed, with_bias=False)
    g = workloads.generator(seed + 1)
    x, r = workloads.activations(M, K, g).cuda(), workloads.activations(M, K, g).cuda()
    w = (0.8 + 0.4 * torch.rand(K, generator=g)).to(torch.bfloat16).cuda()
    ref = torch.ops.paroquant.w4a8_linear_group_rmsnorm(x, r, w, 1e-6, *_lists(mbs), True, True, torch.bfloat16,
                                                        False, False)
    st = ops.W4A8GroupStages(x, *_lists(mbs), x2=r, norm_weight=w, eps=1e-6, mode=_lib.PQ_PRO_RMSNORM)
    st.rotate()
    for y, rr in zip(st.gemm(), ref):
        assert torch.equal(y, rr)


def test_stages_in_separate_graphs():
    """Each stage captured on its own; replays (with eager work between them) give the one-call result."""
    M, K, ns = 1, 4096, (4096, 1024, 1024)
    mbs = _members(ns, K, 8, 515, with_bias=False)
    x = workloads.activations(M, K, workloads.generator(516)).cuda()
    ref = torch.ops.paroquant.w4a8_linear_group(x, *_lists(mbs), True, True, torch.bfloat16)
    st = ops.W4A8GroupStages(x, *_lists(mbs))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        st.rotate()
        st.gemm()
    torch.cuda.current_stream().wait_stream(s)
    g1, g2 = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(g1):
        st.rotate()
    with torch.cuda.graph(g2):
        st.gemm()
    for _ in range(3):
        for y in st.outs:
            y.zero_()
        g1.replay()
        torch.cuda.synchronize()
        junk = torch.randn(1 << 20, device="cuda").sum()   # eager work between the replays
        g2.replay()
        g2.replay()                                        # the GEMM alone again: same workspace, same result
        torch.cuda.synchronize()
        for y, r in zip(st.outs, ref):
            assert torch.equal(y, r)
        del junk


def test_stage_argument_errors():
    mbs = _members((1024,), 4096, 8, 517, with_bias=False)
    x = workloads.activations(2, 4096, workloads.generator(518)).cuda()
    st = ops.W4A8GroupStages(x, *_lists(mbs))
    with pytest.raises(RuntimeError, match="stage 3"):
        st._call(3)
