"""pq_rotation_pack (host C++ in the library): the packed operands carry exactly
the reference's pairs and angles, and the kernels' register-chain use of them
(one cross-lane fetch per layer) is bit-identical to the oracle's rotation."""

import numpy as np
import pytest
import torch

import alpamayo_amd  # noqa: F401
from alpamayo_amd import workloads
from alpamayo_amd.ops import pack_rotation
from oracle import rotation as orot


def _pack(pairs, theta):
    c, s = orot.cos_sin_table(theta.numpy())
    cs = torch.from_numpy(np.stack([c, s], axis=-1)).contiguous()
    idx, rcs = pack_rotation(pairs, cs)
    return idx.numpy(), rcs.numpy(), c, s


def _repeated_perm_params(K, krot, seed):
    """The reference's default initialisation: one randperm(128) for every group and layer
    (rotation_linear.py:32-37), so consecutive layers share every pair."""
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(128, generator=g)
    pairs = perm.repeat(krot, K // 128).to(torch.int16)
    theta = (torch.rand(krot, K // 2, generator=g) * 2 - 1) * np.pi
    return pairs, theta.half()


def _params(kind, K, krot, seed):
    if kind == "random":
        pairs, theta, _ = workloads.rotation_params(K, workloads.generator(seed), krot=krot)
        return pairs, theta
    return _repeated_perm_params(K, krot, seed)


@pytest.mark.parametrize("kind", ["random", "repeated"])
@pytest.mark.parametrize("K,krot", [(128, 8), (4096, 8), (512, 1), (384, 12), (256, 16), (256, 2)])
def test_slot_channels_follow_the_reference_pairs(kind, K, krot):
    """Tracking channel ids through the chain: every layer's lane slots are exactly
    that layer's pairs, with its cosine and the sine negated iff slot A holds the
    pair's second channel; the recorded final channels match."""
    pairs, theta = _params(kind, K, krot, K + krot)
    idx, rcs, c, s = _pack(pairs, theta)
    kp = 8 if krot <= 8 else 16
    G = K // 128
    assert idx.shape == (G, 64, kp // 2) and idx.dtype == np.int32
    assert rcs.shape == (G, 64, kp, 2)
    init, Af, Bf, src, flag, pc, ps = orot.unpack_packed_params(idx, rcs, krot)
    gi, gj = orot.pair_index_arrays(pairs.numpy(), 128)
    lanes = np.arange(64)
    for g in range(G):
        a, b = np.where(init[g], lanes + 64, lanes), np.where(init[g], lanes, lanes + 64)
        for r in range(krot):
            recv = a[src[g, :, r]]
            fl = flag[g, :, r]
            a, b = np.where(fl, recv, b), np.where(fl, b, recv)
            ref = {}
            for t in range(g * 64, g * 64 + 64):
                i, j = gi[r, t] - g * 128, gj[r, t] - g * 128
                ref[(min(i, j), max(i, j))] = (i, c[r, t], s[r, t])
            got = {}
            for lane in range(64):
                key = (min(a[lane], b[lane]), max(a[lane], b[lane]))
                assert key not in got
                got[key] = (a[lane], pc[g, lane, r], ps[g, lane, r])
            assert ref.keys() == got.keys(), f"group {g} layer {r}"
            for key, (first, cc, ss) in ref.items():
                ga, gc, gs = got[key]
                assert gc == cc
                assert gs == (ss if ga == first else -ss)
        np.testing.assert_array_equal(a, Af[g])
        np.testing.assert_array_equal(b, Bf[g])


@pytest.mark.parametrize("kind", ["random", "repeated"])
@pytest.mark.parametrize("K,krot", [(4096, 8), (256, 16), (512, 3), (128, 1)])
def test_kernel_rule_on_packed_operands_is_bit_identical(kind, K, krot):
    pairs, theta = _params(kind, K, krot, 7 * K + krot)
    _, _, scales = workloads.rotation_params(K, workloads.generator(1), krot=krot)
    idx, rcs, c, s = _pack(pairs, theta)
    x = workloads.activations(5, K, workloads.generator(3)).float().numpy()
    xs = orot.scale_rows(x, scales.numpy())
    ref = orot.rotate_f32(xs, pairs.numpy(), c, s, 128)
    got = orot.rotate_f32_packed(xs, idx, rcs, krot)
    np.testing.assert_array_equal(got, ref)


def test_planted_mistake_is_caught():
    """The emulation check is sensitive: one wrong fetch source changes the result."""
    pairs, theta, _ = workloads.rotation_params(256, workloads.generator(9))
    idx, rcs, c, s = _pack(pairs, theta)
    x = workloads.activations(3, 256, workloads.generator(4)).float().numpy()
    ref = orot.rotate_f32(x, pairs.numpy(), c, s, 128)
    bad = idx.copy().view(np.uint8).reshape(2, 64, -1)
    bad[1, 5, 4 + 4] ^= 1                      # layer 4 of lane 5 in group 1 fetches from a neighbour
    got = orot.rotate_f32_packed(x, bad.view(np.uint32).reshape(idx.shape), rcs, 8)
    assert not np.array_equal(got, ref)


def test_pack_rejects_non_matchings():
    pairs, theta, _ = workloads.rotation_params(256, workloads.generator(5))
    bad = pairs.clone()
    bad[2, 7] = bad[2, 9]
    with pytest.raises(ValueError, match="exactly once"):
        _pack(bad, theta)
    bad = pairs.clone()
    bad[0, 0] = 200
    with pytest.raises(ValueError, match="out of"):
        _pack(bad, theta)
