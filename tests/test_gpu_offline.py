"""The offline construction path meets the GPU kernels: weights rotated by rotate_tensor(divide_scale=True)
(rotation_utils.py:32-77) against activations rotated by rotation::rotate keep W' x' = W x, and a layer
built by quantizer -> WQLinear.from_linear -> RotateLinearInt4.from_linear(init_only=False)
(rotation_utils.py:80-97, qmodule.py:149-205, rotation_linear.py:68-118) and converted to W4A8 runs the
fp model's linear to within its quantization error, and the oracle's computation on its codes exactly."""

import pytest
import torch

import alpamayo_amd  # noqa: F401
from alpamayo_amd import workloads
from alpamayo_amd.quantization import (
    BF16RotateLinearWrapper,
    MarlinW4A8Linear,
    RotateLinearInt4,
    convert_model_to_marlin_w4a8,
    rotate_tensor,
)
from oracle import linear as olin
from oracle import packing as opack
from oracle import rotation as orot
from tests.gpu_util import assert_bf16_close, rel_fro, to_np

pytestmark = pytest.mark.gpu


def test_rotated_weights_times_gpu_rotated_activations_keep_the_product():
    K, N = 4096, 96
    pairs, theta, cs = workloads.rotation_params(K, workloads.generator(5100))
    g = workloads.generator(5101)
    w = torch.randn(N, K, generator=g)
    x = torch.randn(7, K, generator=g)
    w_rot = rotate_tensor(w.cuda(), theta.float().cuda(), pairs.cuda(), cs.float().cuda())
    x_rot = torch.ops.rotation.rotate(x.cuda(), pairs.cuda(), theta.float().cuda(), cs.float().cuda(), 128)
    lhs = x_rot.double() @ w_rot.double().t()
    rhs = x.double() @ w.double().t()
    assert rel_fro(to_np(lhs), to_np(rhs)) < 1e-5


@pytest.mark.parametrize("M", [1, 16, 200])
def test_from_linear_layer_converted_to_w4a8(M):
    N, K = 1024, 4096
    g = workloads.generator(5200 + M)
    lin = torch.nn.Linear(K, N, bias=True)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(N, K, generator=g) * 0.02)
        lin.bias.copy_(torch.randn(N, generator=g) * 0.1)
    ref_lin = torch.nn.Linear(K, N, bias=True)
    ref_lin.load_state_dict(lin.state_dict())
    pairs, theta, cs = workloads.rotation_params(K, g)
    rl = RotateLinearInt4.from_linear(lin, rotation_angles=theta, rotation_pairs=pairs, channel_scales=cs,
                                      rotate_weight=True, init_only=False)
    q = rl.qlinear
    awq = opack.wqlinear_to_awq(q.qweight.numpy(), q.scales.numpy(), q.scaled_zeros.numpy(), N, K, 128)
    codes = opack.unpack_wqlinear_qweight(q.qweight.numpy(), N, K)
    bias = q.bias.float().numpy()
    model = torch.nn.Sequential(rl).cuda()
    assert convert_model_to_marlin_w4a8(model) == 1 and isinstance(rl.qlinear, MarlinW4A8Linear)
    x = workloads.activations(M, K, workloads.generator(5300 + M), outlier_frac=0.0)
    y = BF16RotateLinearWrapper(rl)(x.cuda())
    c, s = orot.cos_sin_table(theta.numpy())
    ref, _, _ = olin.w4a8_rotate_linear(to_np(x), pairs.numpy(), c, s, cs.float().numpy().reshape(-1), codes, awq[1],
                                        awq[4], bias)
    assert_bf16_close(to_np(y), ref)
    # the fp model's linear, within the int4 / int8 quantization error
    fp = ref_lin(x.float()).detach().double().numpy()
    assert rel_fro(to_np(y), fp) < 0.25     # about 0.14 from the int4 groups; a wrong rotation gives ~1
