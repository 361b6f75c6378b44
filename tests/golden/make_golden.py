"""Write golden vectors for the functions no closed form or invariant pins.

Run in the build container (it reads the reference sources at
/root/reference, which never travel to the GPU machine):

    python tests/golden/make_golden.py

It imports, by file path, two pure-torch reference functions:

  * ``pack_intweight``  (src/alpamayo_r1/utils/quantization/qmodule.py:39-78):
    the exact WQLinear int16 bit layout;
  * ``pseudo_quantize_tensor`` (src/alpamayo_r1/utils/quantization/
    quantization_utils.py:18-73): the offline uint4 weight quantizer,
    whose rounding ties no invariant pins.

and stores seeded inputs with the reference's outputs in ``golden.npz``
(data only: inputs and expected outputs).
"""

from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np
import torch

REF = "/root/reference/src/alpamayo_r1/utils/quantization"
HERE = os.path.dirname(os.path.abspath(__file__))


def _load(name: str, path: str):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main() -> None:
    qmodule = _load("ref_qmodule", os.path.join(REF, "qmodule.py"))
    qutils = _load("ref_quantization_utils", os.path.join(REF, "quantization_utils.py"))

    out = {}
    g = torch.Generator().manual_seed(20260101)

    # pack_intweight on three shapes (N multiple of 4, K multiple of 64)
    for tag, (N, K) in {"a": (8, 128), "b": (16, 256), "c": (32, 384)}.items():
        codes = torch.randint(0, 16, (N, K), generator=g, dtype=torch.int32)
        packed = qmodule.pack_intweight(codes, interleave=4, kstride=64)
        out[f"pack_{tag}_codes"] = codes.numpy().astype(np.uint8)
        out[f"pack_{tag}_packed"] = packed.numpy()
        zw = qmodule.calculate_zeros_width(K, 128)
        out[f"pack_{tag}_zeros_width"] = np.array([zw], dtype=np.int64)

    # pseudo_quantize_tensor (zero-point branch, 4 bit, group 128)
    for tag, (N, K) in {"a": (16, 256), "b": (8, 512)}.items():
        w = torch.randn(N, K, generator=g, dtype=torch.float32) * 0.05
        w[:, 7] *= 10.0                       # an outlier column
        w_hat, s, z = qutils.pseudo_quantize_tensor(
            w.clone(), n_bit=4, zero_point=True, q_group_size=128, get_scale_zp=True)
        out[f"pq_{tag}_w"] = w.numpy()
        out[f"pq_{tag}_what"] = w_hat.numpy()
        out[f"pq_{tag}_scales"] = s.numpy()
        out[f"pq_{tag}_zeros"] = z.numpy()

    # calculate_zeros_width for the group sizes it accepts
    zw = [(k, gs, qmodule.calculate_zeros_width(k, gs)) for k in (128, 1024, 4096, 12288, 1000 * 128)
          for gs in (32, 64, 128)]
    out["zeros_width_table"] = np.array(zw, dtype=np.int64)

    path = os.path.join(HERE, "golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    sys.exit(main())
