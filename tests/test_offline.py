"""The offline construction path on the CPU (how a ParoQuant checkpoint is made from an fp model):
pseudo_quantize_tensor (quantization_utils.py:18-73), rotate_tensor / apply_rotation_step
(rotation_utils.py:8-77), quantizer (rotation_utils.py:80-97), WQLinear.from_linear (qmodule.py:149-205)
and RotateLinearInt4.from_linear (rotation_linear.py:68-118) -- the product functions, checked against
the golden vectors the reference's own functions wrote, the oracle, and the identities they must meet."""

import numpy as np
import pytest
import torch

import alpamayo_amd  # noqa: F401
from alpamayo_amd import workloads
from alpamayo_amd.quantization import (
    RotateLinearInt4,
    WQLinear,
    dequant_wqlinear,
    pseudo_quantize_tensor,
    quantizer,
    rotate_tensor,
    unpack_wqlinear_qweight,
)
from oracle import rotation as orot


@pytest.mark.parametrize("tag", ["a", "b"])
def test_pseudo_quantize_tensor_matches_golden(golden, tag):
    """The product function gives the reference's w_hat, scales and zeros bit for bit, in all three call forms
    (computed scales, given scales / zeros, in place)."""
    w = torch.from_numpy(golden[f"pq_{tag}_w"].copy())
    what, s, z = pseudo_quantize_tensor(w.clone(), n_bit=4, zero_point=True, q_group_size=128, get_scale_zp=True)
    np.testing.assert_array_equal(what.numpy(), golden[f"pq_{tag}_what"])
    np.testing.assert_array_equal(s.numpy(), golden[f"pq_{tag}_scales"])
    np.testing.assert_array_equal(z.numpy(), golden[f"pq_{tag}_zeros"])
    given = pseudo_quantize_tensor(w.clone(), 4, q_group_size=128, qscales=torch.from_numpy(golden[f"pq_{tag}_scales"]),
                                   qzeros=torch.from_numpy(golden[f"pq_{tag}_zeros"]))
    np.testing.assert_array_equal(given.numpy(), golden[f"pq_{tag}_what"])
    inpl = pseudo_quantize_tensor(w.clone(), n_bit=4, q_group_size=128, inplace=True)
    np.testing.assert_array_equal(inpl.numpy(), golden[f"pq_{tag}_what"])
    with pytest.raises(AssertionError):
        bad = w.clone()
        bad[0, 0] = float("nan")
        pseudo_quantize_tensor(bad, n_bit=4, q_group_size=128)


def _rot_params(K, seed):
    return workloads.rotation_params(K, workloads.generator(seed))


def test_rotate_tensor_multiply_matches_oracle():
    """rotate_tensor(divide_scale=False) is rotation::rotate's math: against the oracle in float32."""
    K = 256
    pairs, theta, cs = _rot_params(K, 11)
    x = torch.randn(6, K, generator=workloads.generator(12))
    got = rotate_tensor(x, theta.float(), pairs, cs.float(), divide_scale=False)
    ref = orot.rotate(x.numpy(), pairs.numpy(), theta.float().numpy(), cs.float().numpy().reshape(-1), 128,
                      out_dtype=np.float32)
    assert np.linalg.norm(got.numpy() - ref) / np.linalg.norm(ref) < 1e-6


def test_rotate_tensor_weights_keep_the_product():
    """Weights rotated with divide_scale=True against activations rotated the kernel's way: W' x' = W x."""
    K, N = 384, 40
    pairs, theta, cs = _rot_params(K, 13)
    w = torch.randn(N, K, generator=workloads.generator(14), dtype=torch.float64).float()
    x = torch.randn(5, K, generator=workloads.generator(15)).float()
    w_rot = rotate_tensor(w, theta.float(), pairs, cs.float())              # rows of W: (R (w / s))
    x_rot = orot.rotate(x.numpy(), pairs.numpy(), theta.float().numpy(), cs.float().numpy().reshape(-1), 128,
                        out_dtype=np.float32)                              # R (s * x)
    lhs = x_rot.astype(np.float64) @ w_rot.double().numpy().T
    rhs = x.double().numpy() @ w.double().numpy().T
    assert np.linalg.norm(lhs - rhs) / np.linalg.norm(rhs) < 1e-5
    assert rotate_tensor(None, theta, pairs, cs) is None


def _quantized_linear(N, K, seed, bias=True):
    g = workloads.generator(seed)
    lin = torch.nn.Linear(K, N, bias=bias)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(N, K, generator=g) * 0.02)
        if bias:
            lin.bias.copy_(torch.randn(N, generator=g) * 0.1)
    return lin


def test_quantizer_builds_the_pseudo_quantized_weights():
    """quantizer -> WQLinear.from_linear stores codes, fp16 scales and scaled zeros whose dequantization is
    pseudo_quantize_tensor's w_hat (the golden-pinned function) up to the fp16 storage of s and -(s z).
    from_linear derives the codes as round((w + z s) / s) in the weights' fp16 arithmetic
    (qmodule.py:185-192), so a few weights near a rounding tie land one code away."""
    N, K = 64, 512
    lin = _quantized_linear(N, K, 21).half()
    w0 = lin.weight.detach().clone()
    q = quantizer(lin, 4, 128)
    assert isinstance(q, WQLinear) and torch.equal(lin.weight, w0)          # the linear is left as it was
    what, s, z = pseudo_quantize_tensor(w0.clone(), n_bit=4, q_group_size=128, get_scale_zp=True)   # in fp16
    what = what.float()
    codes = unpack_wqlinear_qweight(q.qweight, N, K)
    assert int(codes.min()) >= 0 and int(codes.max()) <= 15
    deq = dequant_wqlinear(codes, q.scales, q.scaled_zeros, 128)
    step = s.float().repeat_interleave(128, dim=1)
    off = (deq - what).abs() / step
    assert float((off <= 0.02).float().mean()) >= 0.995
    assert float(off.max()) <= 1.02
    np.testing.assert_array_equal(q.scales[:K // 128].float().numpy(), s.float().t().numpy())
    assert torch.equal(q.bias, lin.bias.detach().half())


def test_rotate_linear_from_linear_quantizes_the_rotated_weights():
    """RotateLinearInt4.from_linear(rotate_weight=True, init_only=False): rotation buffers as given and
    WQLinear weights that dequantize to the rotated weights within half a quantization step."""
    N, K = 48, 256
    pairs, theta, cs = _rot_params(K, 31)
    lin = _quantized_linear(N, K, 32)
    w_rot = rotate_tensor(lin.weight.detach().clone(), theta, pairs, cs)
    rl = RotateLinearInt4.from_linear(lin, rotation_angles=theta, rotation_pairs=pairs, channel_scales=cs,
                                      rotate_weight=True, init_only=False)
    assert torch.equal(rl.rotation.theta, theta) and torch.equal(rl.rotation.pairs, pairs)
    assert torch.equal(rl.rotation.channel_scales, cs)
    assert isinstance(rl.qlinear, WQLinear) and rl.qlinear.qweight.dtype == torch.int16
    codes = unpack_wqlinear_qweight(rl.qlinear.qweight, N, K)
    deq = dequant_wqlinear(codes, rl.qlinear.scales, rl.qlinear.scaled_zeros, 128)
    s = rl.qlinear.scales[:K // 128].float().t().repeat_interleave(128, dim=1)
    assert torch.all((deq - w_rot.float()).abs() <= 0.5 * s + 2e-3 * w_rot.float().abs().max())
    shell = RotateLinearInt4.from_linear(_quantized_linear(N, K, 33), theta, pairs, cs)   # init_only
    assert not shell.qlinear.qweight.any()
