"""Linears that share an input, run as one group (paroquant::w4a8_linear_group,
SharedInputRotateLinears): every member's output against the oracle, and
against a separate paroquant::w4a8_linear call of the same member.  The
reference runs such linears (q/k/v, gate/up) as separate BF16RotateLinearWrapper
calls (paroquant_marlin_w4a8.py:59-65, 455-460); the group must give the same
results."""

import zlib

import pytest
import torch

import alpamayo_amd  # noqa: F401
from alpamayo_amd import workloads
from alpamayo_amd.quantization import SharedInputRotateLinears
from oracle import gemm as ogemm
from oracle import quant as oquant
from oracle import rotation as orot
from tests.gpu_util import assert_bf16_close, packed_rotation, to_np

pytestmark = pytest.mark.gpu


def _members(ns, K, krot, seed, with_bias):
    g = workloads.generator(seed)
    out = []
    for i, N in enumerate(ns):
        spec = workloads.linear_spec(f"m{i}", N, K, g, keep_codes=True)
        pairs = torch.cat([spec.pairs] * 2)[:krot]
        theta = torch.cat([spec.theta] * 2)[:krot]
        rot_idx, rot_cs, c, s = packed_rotation(pairs, theta)
        wp, wm = torch.ops.paroquant.w4a8_prepack(spec.w.awq_qweight.cuda(), spec.w.awq_scales.cuda(),
                                                  spec.w.awq_qzeros.cuda())
        bias = torch.randn(N, generator=g).to(torch.bfloat16) if with_bias and i % 2 == 0 else None
        out.append(dict(spec=spec, pairs=pairs, c=c, s=s, rot_idx=rot_idx.cuda(), rot_cs=rot_cs.cuda(),
                        scales=spec.channel_scales.float().reshape(-1).cuda(), wp=wp, wm=wm,
                        bias=bias.cuda() if bias is not None else None))
    return out


def _oracle(mb, x_np, flags):
    v = orot.rotate_path_f32(x_np, mb["pairs"].numpy(), mb["c"], mb["s"], mb["scales"].cpu().numpy(), 128, *flags)
    q, sx = oquant.quant_int8_per_token(v)
    b = mb["bias"].float().cpu().numpy() if mb["bias"] is not None else None
    return ogemm.w4a8_linear(q, sx, mb["spec"].w.codes.numpy(), mb["spec"].w.awq_scales.numpy(),
                             mb["spec"].w.zeros.numpy(), b)


CASES = [
    # (M, K, member Ns): decode (one kernel pair for all members), the row path, the prefill tiles
    (1, 4096, (4096, 1024, 1024)),
    (1, 4096, (12288, 12288)),
    (3, 4096, (48, 1552, 16, 4096)),
    (1, 12288, (4096,)),
    (4, 12288, (4096, 1024)),
    (9, 12288, (4096, 1040, 16)),
    (24, 12288, (4096, 1024)),   # long rows past 16 tokens: split rotation, token scales, two GEMM row blocks
    (2, 2048, (1024, 64)),
    (5, 4096, (4096, 1024, 1024)),
    (17, 1024, (48, 1552)),
    (300, 4096, (4096, 1024, 1024)),
    (1100, 2048, (1040, 2064, 16)),
    # 192 x 256 tiles past one round: the leading members that fill whole rounds run as a launch of their own
    (1536, 256, (8192, 1024, 1024)),
    (768, 128, (8192, 8192, 2048)),
    (3072, 128, (4096, 1024, 1024)),   # q on 192 x 256 tiles, k/v on 128 x 256 tiles
]


@pytest.mark.parametrize("M,K,ns", CASES)
@pytest.mark.parametrize("krot,flags", [(8, (True, True)), (1, (False, False))])
def test_group_matches_oracle_and_single_calls(M, K, ns, krot, flags):
    print(f"group M={M} K={K} ns={ns} krot={krot} flags={flags}", flush=True)
    seed = zlib.crc32(f"grp{M}-{K}-{ns}-{krot}-{flags}".encode())
    mbs = _members(ns, K, krot, seed, with_bias=True)
    x = workloads.activations(M, K, workloads.generator(seed + 1))
    xc = x.cuda()
    outs = torch.ops.paroquant.w4a8_linear_group(
        xc, [m["rot_idx"] for m in mbs], [m["rot_cs"] for m in mbs], [m["scales"] for m in mbs], krot,
        [m["wp"] for m in mbs], [m["wm"] for m in mbs], [m["bias"] for m in mbs], flags[0], flags[1],
        torch.bfloat16)
    assert len(outs) == len(ns)
    x_np = to_np(x)
    for mb, y, N in zip(mbs, outs, ns):
        assert y.shape == (M, N) and y.dtype == torch.bfloat16
        assert_bf16_close(to_np(y), _oracle(mb, x_np, flags))
        single = torch.ops.paroquant.w4a8_linear(xc, mb["rot_idx"], mb["rot_cs"], mb["scales"], krot, mb["wp"],
                                                 mb["wm"], mb["bias"], flags[0], flags[1], torch.bfloat16)
        if M > 64:
            # same rotate+quant rows, and the prefill tiles accumulate every output element in the same order
            assert torch.equal(y, single)
        else:
            # the decode GEMM (up to 64 rows on int8 A) may split K over a different number of waves for the
            # group
            torch.testing.assert_close(y.float(), single.float(), rtol=2 ** -7, atol=1e-3)


def test_group_output_dtypes_and_leading_dims():
    mbs = _members((64, 128), 1024, 8, 77, with_bias=False)
    x = workloads.activations(6, 1024, workloads.generator(78)).reshape(2, 3, 1024)
    for dt in (torch.float32, torch.float16):
        outs = torch.ops.paroquant.w4a8_linear_group(
            x.cuda().to(dt), [m["rot_idx"] for m in mbs], [m["rot_cs"] for m in mbs], [m["scales"] for m in mbs],
            8, [m["wp"] for m in mbs], [m["wm"] for m in mbs], [None, None], False, True, dt)
        assert [tuple(o.shape) for o in outs] == [(2, 3, 64), (2, 3, 128)] and all(o.dtype == dt for o in outs)
        for mb, y in zip(mbs, outs):
            assert_bf16_close(to_np(y.reshape(6, -1)), _oracle(mb, to_np(x.reshape(6, 1024).to(dt)), (False, True)))


@pytest.mark.parametrize("M", [1, 16, 96])
def test_shared_input_module_matches_members_and_replays(M):
    """SharedInputRotateLinears over q/k/v modules: equal to calling each module, also inside a HIP graph."""
    g = workloads.generator(1209)
    mods = [workloads.build_module(workloads.linear_spec(n, N, 4096, g), "cuda")
            for n, N in (("q_proj", 4096), ("k_proj", 1024), ("v_proj", 1024))]
    grp = SharedInputRotateLinears(mods)
    x = workloads.activations(M, 4096, workloads.generator(1210)).cuda()
    outs = grp(x)
    for mod, y in zip(mods, outs):
        ref = mod(x)
        if M > 16:
            assert torch.equal(y, ref)
        else:
            torch.testing.assert_close(y.float(), ref.float(), rtol=2 ** -7, atol=1e-3)
    eager = [o.clone() for o in outs]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        grp(x)
    torch.cuda.current_stream().wait_stream(s)
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        captured = grp(x)
    for i in range(3):
        gr.replay()
        torch.cuda.synchronize()
        for a, b in zip(captured, eager):
            assert torch.equal(a, b), f"replay {i} differs"
        grp(x)
        torch.cuda.synchronize()


def test_group_rejects_bad_members():
    mbs = _members((64, 128), 1024, 8, 5, with_bias=False)
    x = workloads.activations(2, 1024, workloads.generator(6)).cuda()
    with pytest.raises(Exception, match="1..4"):
        torch.ops.paroquant.w4a8_linear_group(x, [], [], [], 8, [], [], [], True, True, torch.bfloat16)
    other = _members((64,), 2048, 8, 7, with_bias=False)[0]
    with pytest.raises(Exception, match="features"):
        torch.ops.paroquant.w4a8_linear_group(
            x, [mbs[0]["rot_idx"], other["rot_idx"]], [mbs[0]["rot_cs"], other["rot_cs"]],
            [mbs[0]["scales"], other["scales"]], 8, [mbs[0]["wp"], other["wp"]], [mbs[0]["wm"], other["wm"]],
            [None, None], True, True, torch.bfloat16)
