"""pq_w4a8_linear_noalloc (the entry point that allocates nothing) against
pq_w4a8_linear with a caller-owned workspace, through the C ABI: the same
kernels, so the outputs must be identical bit for bit.  Two calls in a row
per case, the second with fewer tokens, so the second call runs on scratch
the first one left behind."""

import ctypes

import pytest
import torch

import alpamayo_amd  # noqa: F401
from alpamayo_amd import _lib, workloads
from tests.gpu_util import packed_rotation

pytestmark = pytest.mark.gpu


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _operands(N, K, seed):
    g = workloads.generator(seed)
    spec = workloads.linear_spec("x", N, K, g)
    rot_idx, rot_cs, _, _ = packed_rotation(spec.pairs, spec.theta)
    wp, wm = torch.ops.paroquant.w4a8_prepack(spec.w.awq_qweight.cuda(), spec.w.awq_scales.cuda(),
                                              spec.w.awq_qzeros.cuda())
    bias = torch.randn(N, generator=g).to(torch.bfloat16).cuda()
    return (rot_idx.cuda(), rot_cs.cuda(), spec.channel_scales.float().reshape(-1).cuda(), wp, wm, bias)


def _run(lib, fn, x, ops, N, K, flags, ws=None):
    rot_idx, rot_cs, sc, wp, wm, bias = ops
    M = x.size(0)
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    common = (x.data_ptr(), _lib.PQ_BF16, rot_idx.data_ptr(), rot_cs.data_ptr(), sc.data_ptr(), wp.data_ptr(),
              wm.data_ptr(), bias.data_ptr(), _lib.PQ_BF16, y.data_ptr(), _lib.PQ_BF16, M, N, K, 8, flags)
    if fn == "noalloc":
        st = lib.pq_w4a8_linear_noalloc(*common, _stream())
    else:
        st = lib.pq_w4a8_linear(*common, ws.data_ptr(), ws.numel(), _stream())
    _lib.check(st, fn)
    return y


# (N, K, first M, second M): the split path (one token), the three-launch long-row path,
# the row rotate+quant path, and a row-path call followed by a split-path call.
CASES = [(4096, 4096, 3, 1), (4096, 12288, 16, 7), (1024, 4096, 700, 96), (12288, 4096, 64, 1)]


@pytest.mark.parametrize("N,K,m1,m2", CASES)
def test_noalloc_matches_workspace_entry_point(N, K, m1, m2):
    print(f"noalloc N={N} K={K} m={m1} then m={m2}", flush=True)
    lib = _lib.load()
    ops = _operands(N, K, 4242 + N + K)
    flags = _lib.PQ_RQ_INPUT_FP16 | _lib.PQ_RQ_MATERIALIZE_FP16
    for M, seed in ((m1, 1), (m2, 2)):
        x = workloads.activations(M, K, workloads.generator(9000 + seed + M)).cuda()
        need = lib.pq_w4a8_linear_workspace_size(M, N, K, 8)
        assert 0 < need <= _lib.PQ_NOALLOC_SCRATCH_BYTES
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        ref = _run(lib, "pq_w4a8_linear", x, ops, N, K, flags, ws)
        got = _run(lib, "noalloc", x, ops, N, K, flags)
        torch.cuda.synchronize()
        assert torch.isfinite(ref.float()).all()
        assert torch.equal(got, ref), f"M={M}: noalloc differs from the workspace entry point"


def test_noalloc_rejects_sizes_beyond_its_scratch():
    lib = _lib.load()
    M, N, K = 3072, 4096, 12288
    assert lib.pq_w4a8_linear_workspace_size(M, N, K, 8) > _lib.PQ_NOALLOC_SCRATCH_BYTES
    p = ctypes.c_void_p(256)
    st = lib.pq_w4a8_linear_noalloc(p, _lib.PQ_BF16, p, p, None, p, p, None, 0, p, _lib.PQ_BF16, M, N, K, 8, 3,
                                    _stream())
    assert _lib.STATUS_NAMES[st] == "PQ_ERR_WORKSPACE"
    assert "scratch" in lib.pq_last_error().decode()
