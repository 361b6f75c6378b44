"""The RMSNorm oracle (oracle/rmsnorm.py) pinned without retyping its formula:
against torch's own rms_norm and bf16 multiply (the library routines of the
reference's Qwen3VLTextRMSNorm.forward, modeling_qwen3_vl.py:354-359), and
by invariants (scale invariance, unit mean square, eps dominance)."""

import numpy as np
import pytest
import torch

from oracle import linear as olin
from oracle import rmsnorm as orms


def _acts(m, k, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g) * 3.0
    x[:, torch.randperm(k, generator=g)[: k // 100]] *= 20.0
    return x.to(torch.bfloat16)


def test_factor_matches_torch_rms_norm_float32():
    x = _acts(8, 4096, 1).float()
    ref = torch.nn.functional.rms_norm(x, (4096,), eps=1e-6).numpy()
    got = x.numpy() * orms.rms_factor(x.numpy(), 1e-6)
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=0)


def test_bf16_semantics_match_torch_reference_ops():
    """h = w * (rms_norm(s) in bf16) in bf16, s = bf16(x + residual), as torch evaluates it."""
    x, res = _acts(16, 4096, 2), _acts(16, 4096, 3)
    w = (0.8 + 0.4 * torch.rand(4096, generator=torch.Generator().manual_seed(4))).to(torch.bfloat16)
    s_t = x + res                                           # bf16 add, as the decoder layer does
    h_t = w * torch.nn.functional.rms_norm(s_t.float(), (4096,), eps=1e-6).to(torch.bfloat16)
    h, s = orms.rmsnorm(x.float().numpy(), w.float().numpy(), 1e-6, res.float().numpy(), "bf16")
    np.testing.assert_array_equal(olin.bf16_bits(s), olin.bf16_bits(s_t.float().numpy()))
    hb, tb = olin.bf16_bits(h).astype(np.int32), olin.bf16_bits(h_t.float().numpy()).astype(np.int32)
    assert np.mean(hb == tb) >= 0.999
    assert np.abs(hb - tb).max() <= 1


def test_scale_invariance_and_unit_mean_square():
    x = _acts(4, 4096, 5).float().numpy()
    w = np.ones(4096, np.float32)
    h1, _ = orms.rmsnorm(x, w, 0.0, dtype="f32")
    h2, _ = orms.rmsnorm(4.0 * x, w, 0.0, dtype="f32")   # a power of two scales exactly
    np.testing.assert_array_equal(h1, h2)
    np.testing.assert_allclose((h1.astype(np.float64) ** 2).mean(-1), 1.0, rtol=1e-6)


def test_eps_dominates_tiny_rows():
    x = np.full((2, 256), 1e-8, np.float32)
    h, _ = orms.rmsnorm(x, np.ones(256, np.float32), 1e-6, dtype="f32")
    np.testing.assert_allclose(h, 1e-8 / np.sqrt(1e-16 + 1e-6), rtol=1e-5)


@pytest.mark.parametrize("dtype,tdt", [("bf16", torch.bfloat16), ("f16", torch.float16)])
def test_swiglu_matches_torch_silu_mul(dtype, tdt):
    """act = silu(g) * u in the module's dtype, against torch's own silu and mul on the CPU."""
    gen = torch.Generator().manual_seed(5150)
    g = (3 * torch.randn(64, 1024, generator=gen)).to(tdt)
    u = torch.randn(64, 1024, generator=gen).to(tdt)
    ref = (torch.nn.functional.silu(g) * u).float().numpy()
    got = orms.swiglu(g.float().numpy(), u.float().numpy(), dtype)
    # a one-ulp difference in silu(g) (float32 exp of numpy vs torch's vector exp) can move the
    # product by up to two ulps of the result: 2^-9 relative for fp16, 2^-6 for bf16
    ulp = np.maximum(np.abs(got), np.abs(ref)).astype(np.float64) * 2.0 ** (-9 if dtype == "f16" else -6)
    diff = np.abs(got.astype(np.float64) - ref)
    assert np.all(diff <= ulp + 6e-8)   # (+ the fp16 subnormal step)
    assert np.mean(diff == 0) >= 0.999


def test_swiglu_special_values():
    g = np.array([0.0, -0.0, 100.0, -100.0, 1e-30], dtype=np.float32)
    u = np.array([5.0, 5.0, 2.0, 2.0, 1.0], dtype=np.float32)
    a = orms.swiglu(g, u, "f32")
    assert a[0] == 0 and a[2] == 200.0 and abs(a[3]) < 1e-40 and a[4] == np.float32(0.5e-30)
