"""GPU parity of rotation::rotate_and_quant_mxfp4 -- the fused rotation + OCP
MXFP4 quantization, the MX counterpart of the reference's NVFP4
rotation::rotate_and_quant (rotation.cu:62-111) -- against the oracle
(oracle/mxfp4.py).

The fused kernel quantizes the float32 rotation result.  rotation::rotate on
float32 copies of the inputs (x, theta and scales converted exactly) yields
that same float32 result, so the codes and scales must equal the oracle's
quantization of it bit for bit (integer/byte work); the float32 rotation
itself is pinned against the oracle by the rotation tests."""

import zlib

import numpy as np
import pytest
import torch

import alpamayo_amd  # noqa: F401
from oracle import mxfp4 as omx
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


def _run(x, pairs, th, sc, gs):
    p = torch.from_numpy(pairs).cuda()
    q, s = torch.ops.rotation.rotate_and_quant_mxfp4(x.cuda(), p, th.cuda(), sc.cuda() if sc is not None else None,
                                                     gs)
    # the float32 rotation the fused kernel quantizes
    y32 = torch.ops.rotation.rotate(x.float().cuda(), p, th.float().cuda(),
                                    sc.float().cuda() if sc is not None else None, gs)
    torch.cuda.synchronize()
    return q.cpu().numpy(), s.cpu().numpy(), to_np(y32)


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("gs,krot,h,rows", [(128, 8, 4096, 5), (128, 1, 256, 1), (64, 4, 192, 33),
                                            (128, 16, 384, 9), (64, 8, 64, 3), (128, 2, 12288, 2),
                                            (128, 8, 4096, 1000), (128, 8, 4096, 1029), (64, 4, 192, 2048)])
@pytest.mark.parametrize("with_scale", [True, False])
def test_mxfp4_matches_oracle(dt, gs, krot, h, rows, with_scale):
    print(f"mxfp4 dt={dt} gs={gs} krot={krot} h={h} rows={rows} scale={with_scale}", flush=True)
    rng = np.random.default_rng(zlib.crc32(f"mx{dt}{gs}{krot}{h}{rows}".encode()))
    pairs, theta, scales = _params(rng, krot, h, gs)
    tdt = DT[dt]
    mag = np.exp2(rng.integers(-12, 12, size=(rows, 1)))   # rows over a range of binades
    x = torch.from_numpy((rng.standard_normal((rows, h)) * mag).astype(np.float32)).to(tdt)
    th = torch.from_numpy(theta).to(tdt)
    sc = torch.from_numpy(scales).to(tdt).reshape(1, h) if with_scale else None
    q, s, y32 = _run(x, pairs, th, sc, gs)
    assert q.shape == (rows, h // 2) and s.shape == (rows, h // 32)
    rq, rs = omx.quantize(y32)
    assert np.array_equal(s, rs), f"{np.sum(s != rs)} scales differ"
    assert np.array_equal(q, rq), f"{np.sum(q != rq)} code bytes differ"
    # and the float32 rotation is the oracle's (to its float32 tolerance)
    ref = orot.rotate(to_np(x), pairs, to_np(th), to_np(sc) if sc is not None else None, gs, out_dtype=np.float32)
    assert rel_fro(y32, ref) < 1e-5
    # dequantized values: MXFP4 noise, at most a quarter of a block's scale step per element on average
    d = omx.dequantize(q, s)
    assert rel_fro(d, ref) < 0.2


def test_mxfp4_special_values_and_leading_dims():
    rng = np.random.default_rng(77)
    h, gs = 256, 128
    pairs, theta, scales = _params(rng, 8, h, gs)
    theta[:] = 0.0                                 # identity rotation: specials stay in place
    x = rng.standard_normal((2, 3, h)).astype(np.float32)
    x[0, 0, :] = 0.0                               # zero row
    x[0, 1, :32] = -0.0
    x[0, 2, 5] = np.nan                            # NaN in block 0
    x[1, 0, 70] = np.inf                           # Inf in block 2
    x[1, 1, :] *= 1e-42                            # subnormal magnitudes
    x[1, 2, :] *= 1e30                             # large magnitudes
    xt = torch.from_numpy(x)
    q, s, y32 = _run(xt, pairs, torch.from_numpy(theta), None, gs)
    assert q.shape == (2, 3, h // 2) and s.shape == (2, 3, h // 32)
    rq, rs = omx.quantize(y32)
    assert np.array_equal(s, rs) and np.array_equal(q, rq)
    assert s[0, 2, 0] == 255 and s[0, 0, 0] == 0 and s[1, 1, 0] == 0


def test_mxfp4_empty_and_checks():
    rng = np.random.default_rng(78)
    pairs, theta, _ = _params(rng, 8, 256, 128)
    x = torch.empty(0, 256, dtype=torch.float16, device="cuda")
    q, s = torch.ops.rotation.rotate_and_quant_mxfp4(x, torch.from_numpy(pairs).cuda(),
                                                     torch.from_numpy(theta).half().cuda(), None, 128)
    assert q.shape == (0, 128) and s.shape == (0, 8)
    with pytest.raises(RuntimeError, match="group_size"):
        torch.ops.rotation.rotate_and_quant_mxfp4(torch.randn(2, 256, device="cuda"), torch.from_numpy(pairs).cuda(),
                                                  torch.from_numpy(theta).cuda(), None, 32)
