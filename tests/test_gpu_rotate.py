"""GPU parity of rotation::rotate (the reference op, rotation.cu:456-493) and
its autograd wrapper (interface.py) against the oracle."""

import zlib

import numpy as np
import pytest
import torch

import alpamayo_amd  # noqa: F401
from alpamayo_amd.paroquant_kernels import scaled_pairwise_rotation
from oracle import rotation as orot
from tests.gpu_util import rel_fro, to_np

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def _params(rng, krot, h, gs):
    pairs = np.concatenate([np.stack([rng.permutation(gs) for _ in range(h // gs)]).reshape(1, -1)
                            for _ in range(krot)]).astype(np.int16)
    theta = rng.uniform(-np.pi, np.pi, (krot, h // 2)).astype(np.float32)
    scales = rng.uniform(0.5, 2, h).astype(np.float32)
    return pairs, theta, scales


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("gs,krot,h,rows", [(128, 8, 4096, 5), (128, 1, 256, 1), (64, 4, 192, 33),
                                            (128, 16, 384, 9), (64, 8, 64, 3), (128, 2, 12288, 2),
                                            (128, 8, 1024, 1030), (64, 16, 320, 2048)])
@pytest.mark.parametrize("with_scale", [True, False])
def test_rotate_matches_oracle(dt, gs, krot, h, rows, with_scale):
    print(f"rotate dt={dt} gs={gs} krot={krot} h={h} rows={rows} scale={with_scale}", flush=True)
    rng = np.random.default_rng(zlib.crc32(f"{dt}{gs}{krot}{h}{rows}".encode()))
    pairs, theta, scales = _params(rng, krot, h, gs)
    tdt = DT[dt]
    x = torch.from_numpy(rng.standard_normal((rows, h)).astype(np.float32) * 3).to(tdt)
    th = torch.from_numpy(theta).to(tdt)
    sc = torch.from_numpy(scales).to(tdt).reshape(1, h) if with_scale else None
    y = torch.ops.rotation.rotate(x.cuda(), torch.from_numpy(pairs).cuda(), th.cuda(),
                                  sc.cuda() if sc is not None else None, gs)
    torch.cuda.synchronize()
    assert y.dtype == tdt and y.shape == x.shape
    ref = orot.rotate(to_np(x), pairs, to_np(th), to_np(sc) if sc is not None else None, gs, out_dtype=np.float32)
    got = to_np(y)
    if dt == "f32":
        assert rel_fro(got, ref) < 1e-5
    else:
        # outputs rounded to fp16/bf16: within one unit of the storage format, plus the float32
        # rounding of the layer chain (cos/sin from sincosf vs the oracle's float64 table, up to
        # ~1e-6 of the row's magnitude after 16 layers), which shows on values near zero
        ulp = 2.0 ** (-10 if dt == "f16" else -7)
        slack = 1e-5 * np.sqrt(np.mean(ref.astype(np.float64) ** 2))
        assert np.all(np.abs(got - ref) <= ulp * np.abs(ref) + slack)
        assert rel_fro(got, ref) < 1e-2


def test_rotate_leading_dims_and_empty():
    rng = np.random.default_rng(1)
    pairs, theta, scales = _params(rng, 8, 256, 128)
    x = torch.randn(2, 3, 256, dtype=torch.float16, device="cuda")
    p = torch.from_numpy(pairs).cuda()
    th = torch.from_numpy(theta).half().cuda()
    y = torch.ops.rotation.rotate(x, p, th, None, 128)
    y2 = torch.ops.rotation.rotate(x.reshape(6, 256), p, th, None, 128)
    assert torch.equal(y.reshape(6, 256), y2)
    e = torch.ops.rotation.rotate(torch.empty(0, 256, dtype=torch.float16, device="cuda"), p, th, None, 128)
    assert e.shape == (0, 256)


def test_rotate_error_paths():
    x = torch.randn(2, 256, dtype=torch.float16, device="cuda")
    p = torch.zeros(8, 256, dtype=torch.int16, device="cuda")
    th = torch.zeros(8, 128, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="Unsupported KROT"):
        torch.ops.rotation.rotate(x, p[:3], th[:3], None, 128)
    with pytest.raises(RuntimeError, match="theta.size"):
        torch.ops.rotation.rotate(x, p[:4], th, None, 128)
    with pytest.raises(RuntimeError, match="group_size"):
        torch.ops.rotation.rotate(x, p, th, None, 32)
    with pytest.raises(RuntimeError, match="dtype"):
        torch.ops.rotation.rotate(x, p, th.float(), None, 128)
    with pytest.raises(RuntimeError, match="only supports"):
        torch.ops.rotation.rotate(x.double(), p, th.double(), None, 128)


def _givens_f64(x, pairs, theta, scale, gs):
    """Differentiable float64 rotation on the CPU (autograd reference)."""
    t = x * scale if scale is not None else x
    h = x.size(-1)
    ng = h // gs
    offs = (torch.arange(ng) * gs)[:, None]
    for r in range(pairs.size(0)):
        p = pairs[r].long().reshape(ng, gs)
        di = (p[:, 0::2] + offs).reshape(-1)
        dj = (p[:, 1::2] + offs).reshape(-1)
        c, s = torch.cos(theta[r]), torch.sin(theta[r])
        a, b = t[:, di], t[:, dj]
        t = t.clone()
        t[:, di] = c * a + s * b
        t[:, dj] = -s * a + c * b
    return t


def test_autograd_backward_matches_float64():
    rng = np.random.default_rng(3)
    h, krot, rows = 256, 8, 6
    pairs, theta, scales = _params(rng, krot, h, 128)
    x64 = torch.from_numpy(rng.standard_normal((rows, h))).requires_grad_(True)
    th64 = torch.from_numpy(theta.astype(np.float64)).requires_grad_(True)
    sc64 = torch.from_numpy(scales.astype(np.float64)).requires_grad_(True)
    w = torch.from_numpy(rng.standard_normal((rows, h)))
    (_givens_f64(x64, torch.from_numpy(pairs), th64, sc64, 128) * w).sum().backward()

    xg = x64.detach().float().cuda().requires_grad_(True)
    thg = th64.detach().float().cuda().requires_grad_(True)
    scg = sc64.detach().float().cuda().requires_grad_(True)
    y = scaled_pairwise_rotation(xg, torch.from_numpy(pairs).cuda(), thg, scg, 128)
    (y * w.float().cuda()).sum().backward()
    assert rel_fro(to_np(xg.grad), x64.grad.numpy()) < 1e-4
    assert rel_fro(to_np(thg.grad), th64.grad.numpy()) < 1e-4
    assert rel_fro(to_np(scg.grad), sc64.grad.numpy()) < 1e-4


_BWD_TOL = {"f32": 2e-6, "f16": 2e-3, "bf16": 1.6e-2}


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("gs,krot,h,rows", [(128, 8, 4096, 5), (128, 1, 256, 1), (64, 4, 192, 33),
                                            (128, 16, 384, 9), (64, 8, 64, 3), (128, 2, 1024, 3000),
                                            (128, 8, 12288, 17), (64, 16, 320, 1030), (128, 8, 256, 0)])
@pytest.mark.parametrize("with_scale", [True, False])
def test_rotate_backward_matches_oracle(dt, gs, krot, h, rows, with_scale):
    """paroquant::rotate_backward (one kernel pass + a fixed-order reduction) against the float64 oracle on
    the same dtype-rounded inputs; 3000 rows exercise the grid-stride row tiles, 0 rows the zero sums."""
    print(f"rotate_backward dt={dt} gs={gs} krot={krot} h={h} rows={rows} scale={with_scale}", flush=True)
    rng = np.random.default_rng(zlib.crc32(f"bwd{dt}{gs}{krot}{h}{rows}".encode()))
    pairs, theta, scales = _params(rng, krot, h, gs)
    tdt = DT[dt]
    x = torch.from_numpy(rng.standard_normal((rows, h)).astype(np.float32) * 3).to(tdt)
    gy = torch.from_numpy(rng.standard_normal((rows, h)).astype(np.float32)).to(tdt)
    th = torch.from_numpy(theta).to(tdt)
    sc = torch.from_numpy(scales).to(tdt).reshape(1, h) if with_scale else None
    idx = torch.from_numpy(pairs)
    gx, gt, gs_ = torch.ops.paroquant.rotate_backward(gy.cuda(), x.cuda(), idx.cuda(), th.cuda(),
                                                      sc.cuda() if sc is not None else None, gs)
    again = torch.ops.paroquant.rotate_backward(gy.cuda(), x.cuda(), idx.cuda(), th.cuda(),
                                                sc.cuda() if sc is not None else None, gs)
    torch.cuda.synchronize()
    assert gx.dtype == tdt and gx.shape == x.shape and gt.dtype == tdt and gt.shape == th.shape
    for a, b in zip((gx, gt, gs_), again):
        assert torch.equal(a, b), "the backward is deterministic"
    rx, rt, rs = orot.rotate_backward(to_np(x).astype(np.float64), pairs, to_np(th),
                                      to_np(sc).reshape(-1) if sc is not None else None,
                                      to_np(gy).astype(np.float64), gs)
    tol = _BWD_TOL[dt]
    if rows == 0:
        assert gx.numel() == 0 and not gt.abs().any()
        if with_scale:
            assert gs_.shape == sc.shape and not gs_.abs().any()
        return
    assert rel_fro(to_np(gx), rx.reshape(x.shape)) < tol
    assert rel_fro(to_np(gt), rt) < tol
    if with_scale:
        assert gs_.shape == sc.shape
        assert rel_fro(to_np(gs_).reshape(-1), rs) < tol
    else:
        assert gs_.numel() == 0


def test_autograd_backward_half_precision_and_no_scale():
    """scaled_pairwise_rotation in fp16 with and without channel scales: gradients against float64 autograd."""
    rng = np.random.default_rng(4)
    h, krot, rows = 512, 8, 40
    pairs, theta, scales = _params(rng, krot, h, 128)
    for with_scale in (True, False):
        x16 = torch.from_numpy(rng.standard_normal((rows, h)).astype(np.float32)).half()
        th16 = torch.from_numpy(theta).half()
        sc16 = torch.from_numpy(scales).half()
        w = torch.from_numpy(rng.standard_normal((rows, h)).astype(np.float32)).half()
        x64 = x16.double().requires_grad_(True)
        th64 = th16.double().requires_grad_(True)
        sc64 = sc16.double().requires_grad_(True)
        (_givens_f64(x64, torch.from_numpy(pairs), th64, sc64 if with_scale else None, 128) * w.double()).sum() \
            .backward()
        xg = x16.cuda().requires_grad_(True)
        thg = th16.cuda().requires_grad_(True)
        scg = sc16.cuda().requires_grad_(True) if with_scale else None
        y = scaled_pairwise_rotation(xg, torch.from_numpy(pairs).cuda(), thg, scg, 128)
        (y * w.cuda()).sum().backward()
        assert rel_fro(to_np(xg.grad), x64.grad.numpy()) < 2e-3
        assert rel_fro(to_np(thg.grad), th64.grad.numpy()) < 2e-3
        if with_scale:
            assert rel_fro(to_np(scg.grad), sc64.grad.numpy()) < 2e-3
