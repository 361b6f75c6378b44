"""ctypes binding of libparoquant_hip.so (the C ABI in include/paroquant_hip.h).

The library is built in-tree by ``alpamayo_amd.build`` (or
``__graft_entry__.build()``).  Loading fails loudly when it is missing:
there is no fallback implementation of any kernel.
"""

from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libparoquant_hip.so")

ABI_VERSION = 1

# enum pq_dtype
PQ_F32, PQ_F16, PQ_BF16 = 0, 1, 2
# flags of pq_rotate_quant_i8
PQ_RQ_INPUT_FP16 = 1
PQ_RQ_MATERIALIZE_FP16 = 2
PQ_PRO_RMSNORM, PQ_PRO_ADD, PQ_PRO_SWIGLU = 1, 2, 3
PQ_ROWS_SAME, PQ_ROWS_MXFP4 = 0, 1
PQ_NOALLOC_SCRATCH_BYTES = 16 << 20

STATUS_NAMES = {0: "PQ_OK", 1: "PQ_ERR_ARG", 2: "PQ_ERR_UNSUPPORTED", 3: "PQ_ERR_HIP", 4: "PQ_ERR_WORKSPACE"}
STATUS_CODE = {v: k for k, v in STATUS_NAMES.items()}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_UINT = ctypes.c_uint
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/paroquant_hip.h
class LinearMember(ctypes.Structure):
    """pq_linear_member: one linear of a group sharing its input (pq_w4a8_linear_group)."""
    _fields_ = [("rot_idx", ctypes.c_void_p), ("rot_cs", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("wpack", ctypes.c_void_p), ("wmeta", ctypes.c_void_p), ("bias", ctypes.c_void_p),
                ("y", ctypes.c_void_p), ("n", ctypes.c_int64)]


MAX_GROUP = 4

SIGNATURES = {
    "pq_abi_version": (_INT, []),
    "pq_last_error": (ctypes.c_char_p, []),
    "pq_rotate": (_INT, [_P, _P, _P, _P, _P, _I64, _I64, _INT, _INT, _INT, _P]),
    "pq_rotate_backward_workspace_size": (_SZ, [_I64, _I64, _INT]),
    "pq_rotate_backward": (_INT, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _INT, _INT, _INT, _P, _SZ, _P]),
    "pq_rotate_mxfp4": (_INT, [_P, _P, _P, _P, _P, _P, _I64, _I64, _INT, _INT, _INT, _P]),
    "pq_rotate_rows": (_INT, [_P, _INT, _P, _P, _P, _P, _P, _I64, _I64, _INT, _INT, _P]),
    "pq_rotate_quant_i8": (_INT, [_P, _INT, _P, _P, _P, _P, _P, _P, _I64, _I64, _INT, _UINT, _P]),
    "pq_quant_i8": (_INT, [_P, _INT, _P, _P, _I64, _I64, _P]),
    "pq_w4a8_workspace_size": (_SZ, [_I64, _I64, _I64, _INT]),
    "pq_w4a8_gemm": (_INT, [_P, _P, _P, _P, _P, _INT, _P, _INT, _I64, _I64, _I64, _INT, _P, _SZ, _P]),
    "pq_w4a8_gemm_partials": (_INT, [_P, _P, _P, _P, _I64, _I64, _I64, _INT, _P]),
    "pq_w4a8_prepack": (_INT, [_P, _P, _P, _P, _P, _I64, _I64, _INT, _P]),
    "pq_rotation_pack": (_INT, [_P, _P, _I64, _INT, _P, _P]),
    "pq_w4a8_linear_workspace_size": (_SZ, [_I64, _I64, _I64, _INT]),
    "pq_w4a8_linear": (_INT, [_P, _INT, _P, _P, _P, _P, _P, _P, _INT, _P, _INT, _I64, _I64, _I64, _INT, _UINT, _P, _SZ,
                              _P]),
    "pq_w4a8_linear_noalloc": (_INT, [_P, _INT, _P, _P, _P, _P, _P, _P, _INT, _P, _INT, _I64, _I64, _I64, _INT, _UINT,
                                      _P]),
    "pq_w4a8_linear_group_workspace_size": (_SZ, [_I64, _I64, _INT]),
    "pq_w4a16_linear_group_workspace_size": (_SZ, [_I64, _I64, _INT]),
    "pq_w4a16_linear_group": (_INT, [_P, _INT, ctypes.POINTER(LinearMember), _INT, _INT, _INT, _I64, _I64, _INT, _UINT,
                                     _P, _SZ, _P]),
    "pq_w4a8_linear_group": (_INT, [_P, _INT, ctypes.POINTER(LinearMember), _INT, _INT, _INT, _I64, _I64, _INT, _UINT,
                                    _P, _SZ, _P]),
    "pq_w4a8_linear_group_rmsnorm": (_INT, [_P, _P, _P, ctypes.c_float, _P, _P, _INT, ctypes.POINTER(LinearMember),
                                            _INT, _INT, _INT, _I64, _I64, _INT, _UINT, _P, _SZ, _P]),
    "pq_w4a8_linear_split_path": (_INT, [_I64, _I64]),
    "pq_w4a8_linear_group_fused": (_INT, [_P, _P, _P, ctypes.c_float, _INT, _P, _P, _INT, ctypes.POINTER(LinearMember),
                                          _INT, _INT, _INT, _I64, _I64, _INT, _UINT, _P, _SZ, _P]),
    "pq_w4a8_linear_group_stage": (_INT, [_INT, _P, _P, _P, ctypes.c_float, _INT, _P, _P, _INT,
                                          ctypes.POINTER(LinearMember), _INT, _INT, _INT, _I64, _I64, _INT, _UINT,
                                          _P, _SZ, _P]),
    "pq_w4a8_linear_group_intermediates": (_INT, [_P, _P, _P, ctypes.c_float, _INT, _P, _P, _INT,
                                                  ctypes.POINTER(LinearMember), _INT, _I64, _I64, _INT, _UINT, _P,
                                                  _SZ, _P, _P, _P, _P]),
    "pq_w4a16_prepack": (_INT, [_P, _P, _P, _P, _P, _I64, _I64, _INT, _P]),
    "pq_w4a16_gemm": (_INT, [_P, _P, _P, _P, _INT, _P, _INT, _I64, _I64, _I64, _INT, _P]),
    "pq_w4a16_linear_workspace_size": (_SZ, [_I64, _I64]),
    "pq_w4a16_linear": (_INT, [_P, _INT, _P, _P, _P, _P, _P, _P, _INT, _P, _INT, _I64, _I64, _I64, _INT, _UINT, _P,
                               _SZ, _P]),
}

_lock = threading.Lock()
_lib = None


class PQError(RuntimeError):
    """A libparoquant_hip entry point returned a non-zero pq_status."""


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it is missing or mismatched."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libparoquant_hip.so not found at {LIB_PATH}; build it with "
                "`python alpamayo_amd/build.py` (there is no non-HIP implementation)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        v = lib.pq_abi_version()
        if v != ABI_VERSION:
            raise RuntimeError(f"libparoquant_hip ABI version {v}, expected {ABI_VERSION}")
        _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().pq_last_error().decode(errors="replace")
        raise PQError(f"{what} failed ({STATUS_NAMES.get(status, status)}): {msg}")
