"""MI355X (gfx950) implementation of the ParoQuant W4A8 linear path.

Layout:
  csrc/               HIP kernels + the C ABI (include/paroquant_hip.h),
                      built into libparoquant_hip.so by build.py
  _lib.py             ctypes binding of the C ABI
  ops.py              torch custom ops (rotation::rotate, paroquant::*)
  paroquant_kernels/  drop-in for the reference's kernels/paroquant_kernels
  quantization/       drop-in for src/alpamayo_r1/utils/quantization
  workloads.py        seeded synthetic inputs of the benchmark configurations

Importing the package loads the HIP library.  On a machine with a GPU a
missing library is an import error; on a CPU-only machine the error is
deferred to the first op call (the ops have no CPU implementation).
"""

import os as _os

import torch as _torch

from . import _lib

if _os.path.exists(_lib.LIB_PATH):
    _lib.load()
elif _torch.cuda.is_available():
    raise ImportError(f"{_lib.LIB_PATH} is missing: build it with `python alpamayo_amd/build.py`")

from . import ops  # noqa: E402,F401

__all__ = ["ops"]
