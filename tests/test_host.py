"""Host-side logic of the package on the CPU: op registration and schemas, fake
kernels, the torch weight-format helpers against the oracle and golden
vectors, module structure against the reference's state-dict keys, and the
absence of any CPU implementation of the kernels."""

import numpy as np
import pytest
import torch

import alpamayo_amd  # noqa: F401  (registers the ops)
from alpamayo_amd import workloads
from alpamayo_amd.quantization import (
    MarlinW4A8Linear,
    RotateLinearInt4,
    Rotation,
    WQLinear,
    check_rotation_pairs,
    pack_awq_int32,
    pack_intweight,
    unpack_awq_int32,
    unpack_wqlinear_qweight,
    wqlinear_to_awq,
)
from oracle import packing


def test_rotate_schema_matches_reference():
    schema = str(torch.ops.rotation.rotate.default._schema)
    assert schema == ("rotation::rotate(Tensor x, Tensor idx_ij, Tensor theta, Tensor? scales, "
                      "int group_size) -> Tensor")


def test_meta_kernels_propagate_shapes():
    m = "meta"
    x = torch.empty(2, 3, 256, device=m, dtype=torch.float16)
    y = torch.ops.rotation.rotate(x, torch.empty(8, 256, device=m, dtype=torch.int16),
                                  torch.empty(8, 128, device=m, dtype=torch.float16), None, 128)
    assert y.shape == x.shape and y.dtype == x.dtype
    xq, xs = torch.ops.paroquant.rotate_quant_i8(x, torch.empty(2, 64, 4, device=m, dtype=torch.int32),
                                                 torch.empty(2, 64, 8, 2, device=m), None, 8, True, True)
    assert xq.shape == (6, 256) and xq.dtype == torch.int8 and xs.shape == (6,)
    wp = torch.empty(64, 2, 64, 16, device=m, dtype=torch.uint8)
    wm = torch.empty(64, 2, 16, device=m, dtype=torch.int32)
    out = torch.ops.paroquant.w4a8_gemm(xq, xs, wp, wm, None, torch.bfloat16)
    assert out.shape == (6, 1024) and out.dtype == torch.bfloat16
    lin = torch.ops.paroquant.w4a8_linear(x, torch.empty(2, 64, 4, device=m, dtype=torch.int32),
                                          torch.empty(2, 64, 8, 2, device=m), None, 8, wp, wm, None, True, True,
                                          torch.bfloat16)
    assert lin.shape == (2, 3, 1024)
    part = torch.ops.paroquant.w4a8_gemm_partials(xq, wp, wm)
    assert part.shape == (6, 2, 1024) and part.dtype == torch.int32


def test_no_cpu_implementation():
    x = torch.zeros(1, 128, dtype=torch.float16)
    with pytest.raises(NotImplementedError):
        torch.ops.rotation.rotate(x, torch.zeros(8, 128, dtype=torch.int16), torch.zeros(8, 64, dtype=torch.float16),
                                  None, 128)
    with pytest.raises(NotImplementedError):
        torch.ops.paroquant.quant_i8(x)


def test_torch_pack_intweight_matches_golden(golden):
    for tag in "abc":
        codes = torch.from_numpy(golden[f"pack_{tag}_codes"].astype(np.int32))
        packed = pack_intweight(codes)
        np.testing.assert_array_equal(packed.numpy(), golden[f"pack_{tag}_packed"])
        np.testing.assert_array_equal(unpack_wqlinear_qweight(packed, *codes.shape).numpy(), codes.numpy())


def test_torch_awq_helpers_match_oracle():
    rng = np.random.default_rng(3)
    v = rng.integers(0, 16, (40, 64)).astype(np.int32)
    t = pack_awq_int32(torch.from_numpy(v))
    np.testing.assert_array_equal(t.numpy(), packing.pack_awq_int32(v))
    np.testing.assert_array_equal(unpack_awq_int32(t, 64).numpy(), v)
    np.testing.assert_array_equal(workloads.pack_awq(torch.from_numpy(v)).numpy(), packing.pack_awq_int32(v))


def test_torch_wqlinear_to_awq_matches_oracle():
    rng = np.random.default_rng(4)
    N, K = 32, 256
    G = K // 128
    codes = rng.integers(0, 16, (N, K)).astype(np.int32)
    zeros = rng.integers(0, 16, (G, N)).astype(np.int32)
    scales = rng.uniform(0.005, 0.02, (G, N)).astype(np.float16)
    zw = packing.calculate_zeros_width(K) * 8
    sc = np.zeros((zw, N), np.float16)
    sc[:G] = scales
    sz = np.zeros((zw, N), np.float16)
    sz[:G] = (-(scales.astype(np.float32) * zeros)).astype(np.float16)
    q16 = packing.pack_intweight(codes)
    ref = packing.wqlinear_to_awq(q16, sc, sz, N, K, 128)
    got = wqlinear_to_awq(torch.from_numpy(q16), torch.from_numpy(sc), torch.from_numpy(sz), N, K, 128)
    for a, b in zip(got, ref):
        np.testing.assert_array_equal(a.numpy(), b)


def test_module_state_dict_keys_match_reference():
    rl = RotateLinearInt4(256, 64, bias=True, dtype=torch.float16)
    keys = set(rl.state_dict().keys())
    assert keys == {"rotation.theta", "rotation.pairs", "rotation.channel_scales", "qlinear.qweight",
                    "qlinear.scales", "qlinear.scaled_zeros", "qlinear.bias"}
    sd = rl.state_dict()
    assert sd["rotation.theta"].shape == (8, 128) and sd["rotation.pairs"].dtype == torch.int16
    assert sd["rotation.channel_scales"].shape == (1, 256)
    assert sd["qlinear.qweight"].shape == (16, 256) and sd["qlinear.qweight"].dtype == torch.int16
    assert sd["qlinear.scales"].shape == (8, 64)
    with pytest.raises(NotImplementedError):
        Rotation(256, krot=4)
    with pytest.raises(NotImplementedError):
        WQLinear(8, 128, 256, 64, False)


def test_rotation_prepare_builds_fused_operands():
    g = workloads.generator(5)
    pairs, theta, cs = workloads.rotation_params(256, g)
    rot = Rotation(256, rotation_angles=theta, rotation_pairs=pairs, channel_scales=cs)
    rot.prepare()
    assert rot.rot_idx.shape == (2, 64, 4) and rot.rot_cs.shape == (2, 64, 8, 2) and rot.krot == 8
    c, s = np.cos(theta.float().double().numpy()), np.sin(theta.float().double().numpy())
    tab = rot.cos_sin_table().numpy()
    np.testing.assert_array_equal(tab[..., 0], c.astype(np.float32))
    np.testing.assert_array_equal(tab[..., 1], s.astype(np.float32))
    np.testing.assert_array_equal(np.sort(np.abs(rot.rot_cs[..., 1].numpy()).ravel()),
                                  np.sort(np.abs(s.astype(np.float32)).ravel()))
    assert "rot_idx" not in rot.state_dict() and "rot_cs" not in rot.state_dict()
    bad = pairs.clone()
    bad[0, 1] = bad[0, 0]
    with pytest.raises(ValueError):
        check_rotation_pairs(bad)


def test_rotation_prepared_tracks_its_parameters():
    """prepared turns False after load_state_dict, an in-place update or a replacement of theta / pairs /
    channel_scales, so the fused paths re-derive their operands instead of using stale ones."""
    g = workloads.generator(6)
    pairs, theta, cs = workloads.rotation_params(256, g)
    rot = Rotation(256, rotation_angles=theta, rotation_pairs=pairs, channel_scales=cs)
    assert not rot.prepared
    rot.prepare()
    assert rot.prepared
    old_cs = rot.rot_cs.clone()
    pairs2, theta2, cs2 = workloads.rotation_params(256, workloads.generator(7))
    rot.load_state_dict({"theta": theta2, "pairs": pairs2, "channel_scales": cs2})
    assert not rot.prepared
    rot.prepare()
    assert rot.prepared and not torch.equal(rot.rot_cs, old_cs)
    rot.channel_scales.mul_(2)
    assert not rot.prepared
    rot.prepare()
    np.testing.assert_array_equal(rot.scales_f32.numpy(), (cs2.float() * 2).reshape(-1).numpy())
    rot.theta = rot.theta.clone()
    assert not rot.prepared


def test_rotate_op_only_looks_up_registered_operands():
    """rotation::rotate never packs: it finds the operands Rotation.prepare() registered for exactly its
    tensors, and the entry lapses when any of them changes."""
    from alpamayo_amd import ops

    g = workloads.generator(8)
    pairs, theta, cs = workloads.rotation_params(256, g)
    rot = Rotation(256, rotation_angles=theta, rotation_pairs=pairs, channel_scales=cs)
    assert ops._packed_for(rot.pairs, rot.theta, rot.channel_scales, 128) is None
    rot.prepare()
    got = ops._packed_for(rot.pairs, rot.theta, rot.channel_scales, 128)
    assert got is not None and got[0] is rot.rot_idx and got[1] is rot.rot_cs
    assert ops._packed_for(rot.pairs.clone(), rot.theta, rot.channel_scales, 128) is None   # other tensor
    assert ops._packed_for(rot.pairs, rot.theta, rot.channel_scales, 64) is None
    th_grad = rot.theta.float().requires_grad_(True)
    assert ops._packed_for(rot.pairs, th_grad, rot.channel_scales, 128) is None
    rot.theta.add_(0.5)
    assert ops._packed_for(rot.pairs, rot.theta, rot.channel_scales, 128) is None


def test_rotate_backward_fake_kernel():
    m = "meta"
    x = torch.empty(3, 5, 256, device=m, dtype=torch.bfloat16)
    idx = torch.empty(8, 256, device=m, dtype=torch.int16)
    th = torch.empty(8, 128, device=m, dtype=torch.bfloat16)
    sc = torch.empty(1, 256, device=m, dtype=torch.bfloat16)
    gx, gt, gs = torch.ops.paroquant.rotate_backward(x, x, idx, th, sc, 128)
    assert gx.shape == x.shape and gt.shape == th.shape and gs.shape == sc.shape and gs.dtype == torch.bfloat16
    gx, gt, gs = torch.ops.paroquant.rotate_backward(x, x, idx, th, None, 128)
    assert gs.numel() == 0


def test_op_implementations_reach_no_host_copy():
    """No op implementation copies to the host or synchronizes (the reference op only enqueues,
    rotation.cu:137): the source of every registered CUDA implementation is free of such calls."""
    import inspect

    from alpamayo_amd import ops

    impls = [v for k, v in vars(ops).items() if k.startswith("_") and k.endswith("_impl") and callable(v)]
    impls += [ops._packed_for, ops._rotate_rows, ops._rotate_args]
    assert len(impls) >= 15
    for fn in impls:
        src = inspect.getsource(fn)
        for bad in ('.to("cpu"', ".cpu()", ".item()", ".tolist()", "synchronize", "pack_rotation(", ".numpy()"):
            assert bad not in src, f"{fn.__name__} contains {bad}"


def test_workloads_are_seeded_and_distributed_as_specified():
    a = workloads.linear_spec("q", 64, 512, workloads.generator(1000), keep_codes=True)
    b = workloads.linear_spec("q", 64, 512, workloads.generator(1000), keep_codes=True)
    assert torch.equal(a.w.awq_qweight, b.w.awq_qweight) and torch.equal(a.theta, b.theta)
    check_rotation_pairs(a.pairs)
    assert a.theta.abs().max() <= np.pi + 1e-3
    cs = a.channel_scales.float()
    assert cs.min() >= 0.5 and cs.max() <= 2.0
    s = a.w.awq_scales.float()
    assert s.min() >= 0.005 and s.max() <= 0.0201
    assert a.w.zeros.min() >= 6 and a.w.zeros.max() <= 9
    x = workloads.activations(16, 4096, workloads.generator(1000))
    assert x.dtype == torch.bfloat16
    big = (x.float().abs().max(dim=0).values > 10).sum().item()
    assert 30 <= big <= 60   # 41 outlier channels (1% of 4096) at x20


def test_marlin_module_requires_load():
    m = MarlinW4A8Linear(256, 64)
    with pytest.raises(RuntimeError, match="load_from_awq"):
        m(torch.zeros(1, 256))
    with pytest.raises(NotImplementedError):
        MarlinW4A8Linear(256, 64, group_size=64)
