"""CPU oracle for the ParoQuant W4A8 linear path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the reference algorithm of every stage of
the path so that the HIP kernels can be checked against it:

  rotation.py  pairwise Givens rotation + channel scale
               (kernels/paroquant_kernels/src/rotation.cuh:247-337,
                rotation.cu:15-60, rotation_utils.py:8-29)
  quant.py     per-token symmetric int8 activation quantization
               (vLLM scaled_int8_quant as invoked by apply_awq_marlin_linear,
                src/alpamayo_r1/utils/quantization/paroquant_marlin_w4a8.py:319-333)
  gemm.py      int4-weight x int8-activation group-scaled GEMM
               (Marlin W4A8 semantics; dequant_awq at paroquant_marlin_w4a8.py:227-235)
  packing.py   WQLinear / AWQ / kernel weight layouts
               (qmodule.py:39-78, paroquant_marlin_w4a8.py:95-209)
  linear.py    the whole linear: rotate -> quant -> GEMM -> bf16
               (paroquant_marlin_w4a8.py:59-65, rotation_linear.py:120-124)
  weightquant.py  offline asymmetric uint4 weight quantizer
               (quantization_utils.py:18-73)
  rmsnorm.py   the decoder layer's RMSNorm (+ residual add) in front of a
               shared-input group (modeling_qwen3_vl.py:354-359)
  mxfp4.py     OCP MXFP4 quantization of the rotated rows (the MX counterpart
               of rotation::rotate_and_quant, rotation.cu:62-111)
  w4a16.py     the W4A16 linear: WQLinear.forward (qmodule.py:207-232) and
               RotateLinearInt4 over it (rotation_linear.py:136-139)

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker: the product
path (``alpamayo_amd``) never imports or calls it and fails loudly when its
HIP library is missing.

Pinning status of each function (how each is checked, see tests/test_oracle_*.py):
  rotation    closed form (explicit float64 block-diagonal matrix product),
              orthogonality / norm invariant, inverse identity (the
              reference's own backward, interface.py:42-50), theta=0 and
              theta=pi/2 special cases, brute-force loop on K=128.
  quant       closed form + invariants (max|q|=127, |q*s-x|<=s/2, sign,
              zero rows).  Tie-breaking (round-half-even) is parity unpinned:
              vLLM is not installed and no reference test pins it.
  gemm        exact int64 brute force of the per-group partials, and a
              float64 dequant_awq matmul for the epilogue.
  rmsnorm     torch.nn.functional.rms_norm (the library routine of the same
              formula) on float32 inputs, scale invariance, unit-weight
              mean(h^2) = 1, eps dominance on tiny rows.
  w4a16       the fp16 weights against the reference's dequant_wqlinear
              formula (float32, exact) rounded once, against dequant_awq
              when sz = -s*z is representable, and a brute-force loop for
              the GEMM.  The external kernels' accumulation order and
              rounding are parity unpinned (not in the reference tree).
  mxfp4       E2M1 grid against the format's bit-level definition, E8M0
              bytes against torch.float8_e8m0fnu, rounding against an
              exhaustive nearest-value search with explicit ties, round trip
              of representable blocks.
  packing     pack_intweight / pseudo_quantize_tensor against golden vectors
              written by importing the reference's own functions in the
              build container (tests/golden/make_golden.py); AWQ order
              against a hand-derived known-answer vector; all inverses by
              round trip.
"""
