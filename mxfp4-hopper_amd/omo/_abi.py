"""Loader of libomo_mxfp4.so, the C ABI declared in include/omo_mxfp4.h.

The library is the only compute path: if it cannot be loaded, importing
``omo`` raises, so nothing can silently fall back to another implementation.
"""
from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "lib", "libomo_mxfp4.so")

OMO_OK = 0
OMO_ERR_INVALID_ARGUMENT = -1
OMO_ERR_UNSUPPORTED = -2
OMO_ERR_HIP = -3

_P, _I64, _I, _F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float

class DualItem(ctypes.Structure):
    """omo_dual_item of include/omo_mxfp4.h."""
    _fields_ = [("input", _P), ("rows", _I64), ("cols", _I64), ("row_q", _P), ("row_q_bytes", _I64),
                ("row_s", _P), ("row_s_bytes", _I64), ("col_q", _P), ("col_q_bytes", _I64), ("col_s", _P),
                ("col_s_bytes", _I64)]


# name -> argtypes, in the order of include/omo_mxfp4.h
SIGNATURES = {
    "omo_hip_per_token_group_quant_fp4": [_P, _I64, _P, _I64, _P, _I64, _I, _F, _F, _F, _I, _P],
    "omo_hip_per_token_Mxfp4ToBf16_dequant": [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _I, _F, _F, _F, _I, _P],
    "omo_hip_per_token_Mxfp4ToFp8": [_P, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _I, _F, _F, _F, _I, _P],
    "omo_hip_per_token_Mxfp4ToBf16ToFp8": [_P, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _I, _F, _F, _F, _I, _P],
    "omo_hip_per_token_Mxfp4ToFp8_col": [_P, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _I, _F, _F, _F, _I, _P],
    "omo_hip_per_token_Mxfp4RowToBf16ToFp8Col": [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _F,
                                                 _P],
    "omo_hip_per_token_Mxfp4RowToBf16ToFp8Col_msplit": [_P, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _P, _P,
                                                        _I64, _I64, _F, _P],
    "omo_hip_quant_mxfp4_dual": [_P, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _F, _P],
    "omo_hip_quant_mxfp4_dual_grouped": [ctypes.POINTER(DualItem), _I64, _F, _P],
    "omo_hip_quant_mxfp4_packed": [_P, _I64, _I64, _P, _I64, _F, _P],
    "omo_hip_packed_Mxfp4ToBf16_dequant": [_P, _I64, _I64, _P, _I64, _P],
    "omo_hip_packed_Mxfp4ToFp8": [_P, _I64, _I64, _P, _I64, _P, _I64, _P],
    "omo_hip_mxfp4_permute_rows": [_P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _P],
    "omo_hip_permute_Mxfp4ToFp8": [_P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _P],
}


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"omo: {LIB_PATH} is missing; build it with `make -C mxfp4-hopper_amd` "
            "(or __graft_entry__.build()). There is no fallback implementation.")
    lib = ctypes.CDLL(LIB_PATH)
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    lib.omo_hip_abi_version.restype = ctypes.c_int
    lib.omo_hip_abi_version.argtypes = []
    lib.omo_hip_last_error.restype = ctypes.c_char_p
    lib.omo_hip_last_error.argtypes = []
    lib.omo_hip_status_string.restype = ctypes.c_char_p
    lib.omo_hip_status_string.argtypes = [ctypes.c_int]
    return lib


lib = _load()


def check(status: int) -> None:
    """Raise the Python error matching a C-ABI status (the reference's
    TORCH_CHECK failures surface as RuntimeError)."""
    if status == OMO_OK:
        return
    msg = lib.omo_hip_last_error().decode(errors="replace")
    if status == OMO_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg or lib.omo_hip_status_string(status).decode())
