"""Drop-in for the reference's ``paroquant_kernels`` package.

Importing it registers ``torch.ops.rotation.rotate`` (schema of
kernels/paroquant_kernels/src/rotation.cu:577) with its fake kernel
(kernels/paroquant_kernels/__init__.py:7-9), backed by the gfx950 HIP
library, and exports the autograd helpers of interface.py.
"""

from .. import ops as _ops  # noqa: F401  (registers the ops)
from .interface import RotateTensorFunc, scaled_pairwise_rotation

__all__ = ["scaled_pairwise_rotation", "RotateTensorFunc"]
