"""The prefill shapes through the modules the benchmark times, against the oracle on row subsets:
all seven Qwen3-8B linears at 3072 tokens one by one, q/k/v and gate/up as groups (one GEMM over 6144 /
24576 concatenated columns), and the ragged packed batch (8 requests of U{1..512} tokens) through the whole
grouped layer (paroquant_marlin_w4a8.py:59-65, 314-333; rotation_linear.py:120-124)."""

import numpy as np
import pytest
import torch

import alpamayo_amd  # noqa: F401
from alpamayo_amd import workloads
from alpamayo_amd.quantization import SharedInputRotateLinears
from oracle import linear as olin
from oracle import rotation as orot
from tests.gpu_util import assert_bf16_close, to_np

pytestmark = pytest.mark.gpu

NAMES = list(workloads.QWEN3_8B_LINEARS)


def _rows(M, seed, extra=10):
    rng = np.random.default_rng(seed)
    fixed = [0, 1, 127, 128, 191, 192, 255, 256, M // 2, M - 2, M - 1]
    return np.unique(np.clip(np.concatenate([fixed, rng.integers(0, M, extra)]), 0, M - 1))


def _oracle(spec, x_np):
    c, s = orot.cos_sin_table(spec.theta.cpu().numpy())
    y, _, _ = olin.w4a8_rotate_linear(x_np, spec.pairs.cpu().numpy(), c, s,
                                      spec.channel_scales.float().cpu().numpy().reshape(-1),
                                      spec.w.codes.cpu().numpy(), spec.w.awq_scales.cpu().numpy(),
                                      spec.w.zeros.cpu().numpy())
    return y


def _layer(seed, dev):
    g = workloads.generator(seed, device=dev)
    specs = [workloads.linear_spec(n, N, K, g, device=dev, keep_codes=True)
             for n, (N, K) in workloads.QWEN3_8B_LINEARS.items()]
    return specs, [workloads.build_module(sp, dev) for sp in specs]


@pytest.mark.parametrize("idx", range(7))
def test_prefill_every_shape_row_subset(idx):
    """Config 2: each of the seven linears alone at 3072 tokens."""
    dev = torch.device("cuda")
    name = NAMES[idx]
    N, K = workloads.QWEN3_8B_LINEARS[name]
    print(f"prefill M=3072 {name} {N}x{K}", flush=True)
    g = workloads.generator(6400 + idx, device=dev)
    spec = workloads.linear_spec(name, N, K, g, device=dev, keep_codes=True)
    mod = workloads.build_module(spec, dev)
    x = workloads.activations(3072, K, g, device=dev)
    y = mod(x)
    rows = _rows(3072, idx)
    assert_bf16_close(to_np(y)[rows], _oracle(spec, to_np(x)[rows]))


def test_prefill_groups_row_subset():
    """Config 2 as the benchmark runs it: q/k/v as one group (GEMM over 6144 columns) and gate/up as one
    group (24576 columns), each member against the oracle."""
    dev = torch.device("cuda")
    specs, mods = _layer(6500, dev)
    g = workloads.generator(6501, device=dev)
    xa = workloads.activations(3072, 4096, g, device=dev)
    xm = workloads.activations(3072, 4096, g, device=dev)
    rows = _rows(3072, 6502)
    for members, x, idxs in ((mods[0:3], xa, (0, 1, 2)), (mods[4:6], xm, (4, 5))):
        outs = SharedInputRotateLinears(members)(x)
        xr = to_np(x)[rows]
        for y, i in zip(outs, idxs):
            print(f"prefill group member {NAMES[i]}", flush=True)
            assert y.shape == (3072, specs[i].N)
            assert_bf16_close(to_np(y)[rows], _oracle(specs[i], xr))


def test_ragged_batch_whole_layer():
    """Config 4: 8 requests of U{1..512} tokens (seed 1004) packed without padding through the grouped layer
    (q/k/v, o, gate/up, down); every shape against the oracle on rows of every request, and each request's
    rows equal to that request run alone (per-row quantization) up to the GEMM's summation order (a short
    request alone runs the decode kernels)."""
    dev = torch.device("cuda")
    lens = workloads.ragged_lengths(8, workloads.generator(1004))
    offs = np.concatenate([[0], np.cumsum(lens)])
    M = int(offs[-1])
    specs, mods = _layer(6600, dev)
    qkv, gu = SharedInputRotateLinears(mods[0:3]), SharedInputRotateLinears(mods[4:6])
    g = workloads.generator(6601, device=dev)
    X = [workloads.activations(M, K, g, device=dev) for K in (4096, 4096, 4096, 12288)]

    def layer(xa, xo, xm, xd):
        return [*qkv(xa), mods[3](xo), *gu(xm), mods[6](xd)]

    outs = layer(*X)
    inputs = (X[0], X[0], X[0], X[1], X[2], X[2], X[3])
    rows = np.unique(np.concatenate([[offs[r], offs[r + 1] - 1] for r in range(8)] +
                                    [np.random.default_rng(7).integers(0, M, 8)]))
    for i, (y, x) in enumerate(zip(outs, inputs)):
        print(f"ragged M={M} {NAMES[i]}", flush=True)
        assert_bf16_close(to_np(y)[rows], _oracle(specs[i], to_np(x)[rows]))
    for r in range(8):
        a, b = int(offs[r]), int(offs[r + 1])
        alone = layer(*(x[a:b] for x in X))
        for i, (y, ya) in enumerate(zip(outs, alone)):
            assert_bf16_close(to_np(ya), to_np(y[a:b]).astype(np.float64))
