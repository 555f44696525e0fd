"""ctypes binding of ``libqdc_hip.so`` (declared in ``include/qdc_hip.h``).

The library is loaded from ``qwendecisioncore.jl_amd/lib/`` (built in-tree by
``make -C qwendecisioncore.jl_amd/csrc``).  There is no fallback: a missing
library is an error.  Status codes map to exceptions the way the reference maps
bad input to ``ArgumentError`` / ``DimensionMismatch``: a negative status raises
``ValueError`` (argument error found on the host before any launch), a positive
one ``RuntimeError`` (HIP launch failure).
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "lib", "libqdc_hip.so")

QDC_F32 = 0
QDC_BF16 = 1
QDC_BF16X2 = 2  # output only: two bf16 terms per fp32 value

STATUS = {0: "QDC_OK", -1: "QDC_ERR_NULL", -2: "QDC_ERR_SHAPE", -3: "QDC_ERR_DTYPE",
          -4: "QDC_ERR_RANGE", -5: "QDC_ERR_ALIAS"}

_i32, _i64, _f32, _vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p

# name -> (restype, argtypes); the order of declarations in include/qdc_hip.h
SIGNATURES = {
    "qdc_version": (ctypes.c_char_p, []),
    "qdc_status_string": (ctypes.c_char_p, [_i32]),
    "qdc_embedding_gather": (_i32, [_vp, _i32, _vp, _i32, _vp, _i64, _i64, _i64, _vp, _vp]),
    "qdc_embedding_gather_rmsnorm": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _i32, _vp, _i64, _i64,
                                            _i64, _f32, _vp, _vp]),
    "qdc_check_ids": (_i32, [_vp, _i64, _i64]),
    "qdc_rmsnorm": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _i32, _i32, _i32, _vp]),
    "qdc_residual_rmsnorm": (_i32, [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32, _i32, _i32, _i32,
                                    _vp]),
    "qdc_rmsnorm_masked": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _i32, _i32,
                                  _i32, _vp]),
    "qdc_residual_rmsnorm_masked": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32, _i32,
                                           _i32, _i32, _vp]),
    "qdc_qk_norm_rope": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp] + [_i64] * 16
                         + [_f32, _i32, _vp]),
    "qdc_qk_norm_rope_batched": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp] + [_i64] * 18
                                 + [_f32, _i32, _vp]),
    "qdc_attention_prepare": (_i32, [_vp] * 10 + [_i64] * 12 + [_f32, _i32, _vp]),
    "qdc_rope_tables": (_i32, [_vp, _vp, _i64, _i64, _f32]),
    "qdc_gated_rmsnorm": (_i32, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _f32,
                                 _i32, _i32, _vp]),
    "qdc_swiglu": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i32, _i32, _vp]),
    "qdc_delta_scan": (_i32, [_vp, _i32, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                              _i64, _i64, _i64, _vp]),
    "qdc_delta_prologue": (_i32, [_vp, _vp, _vp, _vp, _vp, _vp, _i32, _i64, _vp, _i64, _vp, _vp,
                                  _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp]),
    "qdc_attention_softmax": (_i32, [_vp, _i32, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _f32,
                                     _vp]),
    "qdc_attention_gate": (_i32, [_vp, _i32, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _i64,
                                  _i64, _vp]),
    "qdc_copy": (_i32, [_vp, _vp, _i64, _vp]),
    "qdc_copy_grid": (_i32, [_vp, _vp, _i64, _i32, _i32, _vp]),
    "qdc_copy_pair": (_i32, [_vp, _vp, _i64, _vp, _vp, _i64, _i32, _i32, _vp]),
    "qdc_copy_rows": (_i32, [_vp, _vp, _vp, _i64, _i64, _i64, _i32, _vp]),
    "qdc_empty": (_i32, [_i64, _vp]),
    "qdc_row_scale": (_i32, [_vp, _vp, _i64, _f32, _f32, _vp]),
    "qdc_row_scale_check": (_i32, [ctypes.c_uint32, _i64, _vp, _vp]),
}

_lib = None


class QDCError(RuntimeError):
    """A HIP launch failure reported by the library (positive status)."""


def lib():
    """The loaded library (loads it on first use)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `make -C qwendecisioncore.jl_amd/csrc` "
                "or __graft_entry__.build()")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def status_string(status: int) -> str:
    return lib().qdc_status_string(status).decode()


def check(status: int, what: str) -> None:
    """Raise for a non-zero status returned by entry point ``what``."""
    if status == 0:
        return
    text = status_string(status)
    if status < 0:
        raise ValueError(f"{what}: {STATUS.get(status, status)}: {text}")
    raise QDCError(f"{what}: hipError {status}: {text}")


def version() -> str:
    return lib().qdc_version().decode()
