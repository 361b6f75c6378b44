"""The packed-operand rotation (pq_rotate_rows: the fused linear's register-chain
kernel with a plain or MXFP4 output) against the LDS-tile kernel of
rotation::rotate / rotate_and_quant_mxfp4 (pq_rotate, pq_rotate_mxfp4) on the
same inputs: both take cos/sin of each stored angle in float64, rounded once,
and apply the layers in the same float32 order, so the outputs must be equal
bit for bit.  Also: the ops pick the packed kernel from 1024 rows on, in and
out of graph capture, and recompute the operands when the angles change."""

import zlib

import numpy as np
import pytest
import torch

import alpamayo_amd  # noqa: F401
from alpamayo_amd import _lib, ops
from alpamayo_amd.ops import pack_rotation
from oracle import mxfp4 as omx
from oracle import rotation as orot
from tests.gpu_util import rel_fro, to_np

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def _params(rng, krot, h):
    pairs = np.concatenate([np.stack([rng.permutation(128) for _ in range(h // 128)]).reshape(1, -1)
                            for _ in range(krot)]).astype(np.int16)
    theta = rng.uniform(-np.pi, np.pi, (krot, h // 2)).astype(np.float32)
    scales = rng.uniform(0.5, 2, h).astype(np.float32)
    return pairs, theta, scales


def _tile(fn, *args):
    lib = _lib.load()
    st = getattr(lib, fn)(*args)
    assert st == 0, lib.pq_last_error().decode()


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("krot,h,rows", [(8, 4096, 5), (1, 128, 3), (16, 384, 33), (2, 12288, 17), (8, 4096, 1029)])
@pytest.mark.parametrize("with_scale", [True, False])
def test_packed_kernel_equals_tile_kernel(dt, krot, h, rows, with_scale):
    print(f"rotate_rows dt={dt} krot={krot} h={h} rows={rows} scale={with_scale}", flush=True)
    rng = np.random.default_rng(zlib.crc32(f"rr{dt}{krot}{h}{rows}{with_scale}".encode()))
    pairs, theta, scales = _params(rng, krot, h)
    tdt = DT[dt]
    x = torch.from_numpy(rng.standard_normal((rows, h)).astype(np.float32) * 3).to(tdt).cuda()
    th = torch.from_numpy(theta).to(tdt)
    sc = torch.from_numpy(scales).to(tdt) if with_scale else None
    p = torch.from_numpy(pairs).cuda()
    thd = th.cuda()
    scd = sc.cuda() if sc is not None else None
    # packed operands exactly as the op derives them
    cs = torch.stack([torch.cos(th.double()), torch.sin(th.double())], dim=-1).float()
    rot_idx, rot_cs = pack_rotation(torch.from_numpy(pairs), cs)
    rot_idx, rot_cs = rot_idx.cuda(), rot_cs.cuda()
    sf = scd.float().contiguous() if scd is not None else None
    dtc = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[tdt]
    y_tile, y_rows = torch.empty_like(x), torch.empty_like(x)
    _tile("pq_rotate", x.data_ptr(), y_tile.data_ptr(), p.data_ptr(), thd.data_ptr(),
          scd.data_ptr() if scd is not None else None, rows, h, krot, 128, dtc, None)
    _tile("pq_rotate_rows", x.data_ptr(), dtc, rot_idx.data_ptr(), rot_cs.data_ptr(),
          sf.data_ptr() if sf is not None else None, y_rows.data_ptr(), None, rows, h, krot, _lib.PQ_ROWS_SAME, None)
    q_tile = torch.empty((rows, h // 2), dtype=torch.uint8, device="cuda")
    s_tile = torch.empty((rows, h // 32), dtype=torch.uint8, device="cuda")
    q_rows, s_rows = torch.empty_like(q_tile), torch.empty_like(s_tile)
    _tile("pq_rotate_mxfp4", x.data_ptr(), q_tile.data_ptr(), s_tile.data_ptr(), p.data_ptr(), thd.data_ptr(),
          scd.data_ptr() if scd is not None else None, rows, h, krot, 128, dtc, None)
    _tile("pq_rotate_rows", x.data_ptr(), dtc, rot_idx.data_ptr(), rot_cs.data_ptr(),
          sf.data_ptr() if sf is not None else None, q_rows.data_ptr(), s_rows.data_ptr(), rows, h, krot,
          _lib.PQ_ROWS_MXFP4, None)
    torch.cuda.synchronize()
    assert torch.equal(y_rows.view(torch.int16 if dt != "f32" else torch.int32),
                       y_tile.view(torch.int16 if dt != "f32" else torch.int32))
    assert torch.equal(q_rows, q_tile) and torch.equal(s_rows, s_tile)
    # and against the oracle
    ref = orot.rotate(to_np(x), pairs, to_np(th), to_np(sc) if sc is not None else None, 128, out_dtype=np.float32)
    assert rel_fro(to_np(y_rows), ref) < (1e-5 if dt == "f32" else 1e-2)


def test_ops_use_registered_packed_operands_from_1024_rows_and_in_graphs():
    """rotation::rotate / rotate_and_quant_mxfp4 on a prepared Rotation's own buffers run the packed-operand
    kernel from 1024 rows (the operands Rotation.prepare() registered; the op never packs); the same values
    in other tensors run the tile kernel; both give the same bits.  An in-place update of the angles lapses
    the registration until the next prepare()."""
    from alpamayo_amd.quantization import Rotation

    rng = np.random.default_rng(99)
    h, krot = 4096, 8
    pairs, theta, scales = _params(rng, krot, h)
    p = torch.from_numpy(pairs).cuda()
    th = torch.from_numpy(theta).bfloat16().cuda()
    sc = torch.from_numpy(scales).bfloat16().cuda().reshape(1, h)
    rot = Rotation(h, rotation_angles=th, rotation_pairs=p, channel_scales=sc).cuda()
    rot.prepare()
    x = torch.randn(2048, h, device="cuda").bfloat16()
    assert ops._packed_for(rot.pairs, rot.theta, rot.channel_scales, 128) is not None
    y = rot(x)                                                      # packed kernel
    y_tile = torch.ops.rotation.rotate(x, p.clone(), th.clone(), sc.clone(), 128)   # unregistered: tile kernel
    assert ops._packed_for(p, th, sc, 128) is None
    assert torch.equal(y, y_tile)
    q, s = torch.ops.rotation.rotate_and_quant_mxfp4(x, rot.pairs, rot.theta, rot.channel_scales, 128)
    y32 = torch.ops.rotation.rotate(x.float(), p, th.float(), sc.float(), 128)
    rq, rs = omx.quantize(to_np(y32))
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(s.cpu().numpy(), rs)
    small = rot(x[:16])                                             # tile kernel below 1024 rows
    assert torch.equal(small, y[:16])
    # graph capture replays the packed kernel
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        rot(x)
    torch.cuda.current_stream().wait_stream(st)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        yc = rot(x)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yc, y)
    # new angles (in-place update): the registration lapses (tile kernel, new values) until prepare()
    rot.theta.mul_(0.5)
    assert not rot.prepared and ops._packed_for(rot.pairs, rot.theta, rot.channel_scales, 128) is None
    y2 = rot(x)
    ref2 = orot.rotate(to_np(x), pairs, to_np(rot.theta), to_np(sc), 128, out_dtype=np.float32)
    assert rel_fro(to_np(y2), ref2) < 1e-2 and not torch.equal(y2, y)
    rot.prepare()
    assert torch.equal(rot(x), y2)
