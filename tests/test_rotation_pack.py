"""pq_rotation_pack (host C++ in the library): the packed operands carry exactly
the reference's pairs and angles, the kernels' way of applying them is bit-identical
to the oracle's rotation, and every layer's LDS accesses are bank-conflict free."""

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
    ij, rcs = pack_rotation(pairs, cs)
    return ij.numpy(), rcs.numpy(), c, s


@pytest.mark.parametrize("K,krot", [(128, 8), (4096, 8), (512, 1), (384, 12), (256, 16)])
def test_packed_operands_hold_the_same_rotation(K, krot):
    pairs, theta, _ = workloads.rotation_params(K, workloads.generator(K + krot), krot=krot)
    ij, rcs, c, s = _pack(pairs, theta)
    kp = (krot + 7) // 8 * 8
    assert ij.shape == (K // 128, 64, kp) and rcs.shape == (K // 128, 64, kp, 2)
    first, second, pc, ps = orot.unpack_packed_params(ij, rcs, krot)
    gi, gj = orot.pair_index_arrays(pairs.numpy(), 128)
    for r in range(krot):
        ref = {}
        for t in range(K // 2):
            g = t // 64
            ref[(g, min(gi[r, t], gj[r, t]) - g * 128, max(gi[r, t], gj[r, t]) - g * 128)] = \
                (gi[r, t] - g * 128, c[r, t], s[r, t])
        got = {}
        for g in range(K // 128):
            for lane in range(64):
                a, b = int(first[g, lane, r]), int(second[g, lane, r])
                got[(g, min(a, b), max(a, b))] = (a, pc[g, lane, r], ps[g, lane, r])
        assert ref.keys() == got.keys()
        for key, (fa, cc, ss) in ref.items():
            ga, gc, gs = got[key]
            assert gc == cc
            assert gs == (ss if ga == fa else -ss)      # swapped pair <=> negated sine


@pytest.mark.parametrize("K,krot", [(4096, 8), (256, 16), (512, 3)])
def test_kernel_rule_on_packed_operands_is_bit_identical(K, krot):
    pairs, theta, scales = workloads.rotation_params(K, workloads.generator(7 * K + krot), krot=krot)
    ij, rcs, c, s = _pack(pairs, theta)
    x = workloads.activations(5, K, workloads.generator(3)).float().numpy()
    xs = orot.scale_rows(x, scales.numpy())
    ref = orot.rotate_f32(xs, pairs.numpy(), c, s, 128)
    got = orot.rotate_f32_packed(xs, ij, rcs, krot)
    np.testing.assert_array_equal(got, ref)


def test_lds_banks_conflict_free():
    pairs, theta, _ = workloads.rotation_params(4096, workloads.generator(11))
    ij, rcs, _, _ = _pack(pairs, theta)
    first, second, _, _ = orot.unpack_packed_params(ij, rcs, 8)
    for half in (slice(0, 32), slice(32, 64)):
        for arr in (first, second):
            banks = arr[:, half, :] & 31                    # [G, 32, krot]
            srt = np.sort(banks, axis=1)
            assert np.array_equal(srt, np.broadcast_to(np.arange(32)[None, :, None], srt.shape))


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
