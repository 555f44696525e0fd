"""numpy front end of the CPU oracle (``oracle/liboracle.so``).

TEST INFRASTRUCTURE ONLY.  These functions restate the reference's CPU path for
the fused row kernels and are what the HIP library is compared with; only
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
call them.  Nothing in the product package imports this module.

Arrays are row-major numpy arrays: ``[rows, width]`` here is the reference's
column-major ``(width, rows)``.  Every function takes and returns float32 (or
uint16 bf16 bit patterns for the format helpers); bf16 inputs are widened with
:func:`bf16_to_f32` by the caller, exactly as the reference widens at load
(``src/safetensors.jl:28-30``).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64 = ctypes.c_int64


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        raise RuntimeError(f"CPU oracle not built: {_LIB_PATH} (run `make -C oracle`)")
    lib = ctypes.CDLL(_LIB_PATH)
    lib.qdco_bf16_to_f32_n.argtypes = [_u16p, _f32p, _i64]
    lib.qdco_f32_to_bf16_n.argtypes = [_f32p, _u16p, _i64]
    lib.qdco_gather.argtypes = [ctypes.c_void_p, ctypes.c_void_p, _i64, _i32p, _i64, _i64, _i64]
    lib.qdco_gather.restype = ctypes.c_int
    lib.qdco_rms.argtypes = [_f32p, _i64, _f32p, _i64, _f32p, _i64, _i64, ctypes.c_float, ctypes.c_int]
    lib.qdco_residual_rms.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _i64, _i64, ctypes.c_float]
    lib.qdco_rope_tables.argtypes = [_f32p, _f32p, _i64, _i64, ctypes.c_float]
    lib.qdco_qk_norm_rope.argtypes = [_f32p, _i64, _i64, _f32p, _i64, _i64, _f32p, _f32p, _f32p,
                                      _i64, _i64, _i64, _i64, _i64, _i64, ctypes.c_float]
    lib.qdco_gated_rms.argtypes = [_f32p, _i64, _f32p, _i64, _f32p, _i64, _f32p, _i64, _i64, _i64,
                                   ctypes.c_float]
    lib.qdco_swiglu.argtypes = [_f32p, _i64, _f32p, _i64, _f32p, _i64, _i64, _i64]
    lib.qdco_set_threads.argtypes = [ctypes.c_int]
    lib.qdco_threads.restype = ctypes.c_int
    _lib = lib
    return lib


def set_threads(threads: int) -> int:
    """Threads for the C row loops (1 by default; results do not depend on it).
    Returns the previous count."""
    lib = _load()
    previous = lib.qdco_threads()
    lib.qdco_set_threads(int(threads))
    return previous


def _p(a, t=_f32p):
    return a.ctypes.data_as(t)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """Widen bf16 bit patterns: ``src/safetensors.jl:28-30``."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    _load().qdco_bf16_to_f32_n(_p(bits, _u16p), _p(out), bits.size)
    return out


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round to bf16 bit patterns, RNE: ``src/safetensors.jl:37-42``."""
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    _load().qdco_f32_to_bf16_n(_p(x), _p(out, _u16p), x.size)
    return out


def round_bf16(x: np.ndarray) -> np.ndarray:
    """fp32 values made bf16-representable (narrow, then widen)."""
    return bf16_to_f32(f32_to_bf16(x))


def split_bf16(x: np.ndarray) -> np.ndarray:
    """The two-term bf16 form of fp32 values (the library's ``QDC_BF16X2`` output;
    no counterpart in the reference, whose GPU path is fp32 only): ``hi = bf16(x)``
    and ``lo = bf16(x - hi)``, both RNE as :func:`f32_to_bf16`, ``lo = 0`` where
    ``hi`` is not finite.  Returns uint16 bit patterns ``[..., 2K]`` for ``[..., K]``
    (K a multiple of 4), every aligned group of 4 elements laid out ``[4 hi | 4 lo]``."""
    x = _f32(x)
    K = x.shape[-1]
    if K % 4:
        raise ValueError("the split form needs whole groups of 4 elements")
    hi_bits = f32_to_bf16(x)
    hi = bf16_to_f32(hi_bits)
    with np.errstate(invalid="ignore"):
        rest = np.where(np.isfinite(hi), x - hi, np.float32(0)).astype(np.float32)
    lo_bits = f32_to_bf16(rest)
    lead = x.shape[:-1]
    pieces = np.stack([hi_bits.reshape(*lead, K // 4, 4), lo_bits.reshape(*lead, K // 4, 4)], -2)
    return pieces.reshape(*lead, 2 * K)


def join_split(bits: np.ndarray) -> np.ndarray:
    """fp32 ``hi + lo`` of split bit patterns ``[..., 2K]`` -> ``[..., K]``."""
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    lead, K2 = bits.shape[:-1], bits.shape[-1]
    g = bf16_to_f32(bits).reshape(*lead, K2 // 8, 2, 4)
    return (g[..., 0, :] + g[..., 1, :]).astype(np.float32).reshape(*lead, K2 // 2)


def round_split(x: np.ndarray) -> np.ndarray:
    """fp32 values as the split form stores them (``hi + lo``)."""
    return join_split(split_bf16(x))


def gather(table: np.ndarray, ids: np.ndarray) -> np.ndarray:
    """``src/backbone.jl:56-64``: row copy, any element type.  ValueError on a bad id."""
    table = np.ascontiguousarray(table)
    ids = np.ascontiguousarray(ids, dtype=np.int32).reshape(-1)
    vocab, hidden = table.shape
    out = np.empty((ids.size, hidden), table.dtype)
    rc = _load().qdco_gather(out.ctypes.data, table.ctypes.data, table.itemsize, _p(ids, _i32p),
                             ids.size, vocab, hidden)
    if rc != 0:
        raise ValueError("Token ID is outside the vocabulary.")
    return out


def rms(x: np.ndarray, w: np.ndarray, eps: float, centered: bool = True) -> np.ndarray:
    """``cpu_rms!`` (centred) / ``cpu_delta_rms!`` over the last axis."""
    x = _f32(x)
    w = _f32(w)
    width = x.shape[-1]
    rows = x.size // width if width else 0
    out = np.empty_like(x)
    _load().qdco_rms(_p(out), width, _p(x), width, _p(w), rows, width, eps, int(centered))
    return out


def residual_rms(x: np.ndarray, mixed: np.ndarray, w: np.ndarray, eps: float):
    """``native_residual_rms``: returns ``(x + mixed, rms(x + mixed))``."""
    x, mixed, w = _f32(x), _f32(mixed), _f32(w)
    width = x.shape[-1]
    rows = x.size // width if width else 0
    residual = np.empty_like(x)
    out = np.empty_like(x)
    _load().qdco_residual_rms(_p(residual), _p(out), _p(x), _p(mixed), _p(w), rows, width, eps)
    return residual, out


def rope_tables(n_pos: int, rotary_dim: int, theta: float):
    """``cpu_full_workspace`` tables, each ``[n_pos, rotary_dim // 2]`` fp32."""
    half = rotary_dim // 2
    cos = np.empty((n_pos, half), np.float32)
    sin = np.empty((n_pos, half), np.float32)
    _load().qdco_rope_tables(_p(cos), _p(sin), n_pos, rotary_dim, theta)
    return cos, sin


def qk_norm_rope(x: np.ndarray, w: np.ndarray, cos: np.ndarray, sin: np.ndarray, rotary_dim: int,
                 eps: float, seq_len: int | None = None, pos_offset: int = 0) -> np.ndarray:
    """Per-head centred RMSNorm then partial RoPE on ``x [tokens, heads, dim]``.

    ``cpu_full_rms!`` + ``cpu_full_rope!``; token ``t`` sits at position
    ``pos_offset + t % seq_len`` in the tables."""
    x = _f32(x)
    tokens, heads, dim = x.shape
    seq_len = tokens if seq_len is None else seq_len
    cos, sin, w = _f32(cos), _f32(sin), _f32(w)
    out = np.empty_like(x)
    _load().qdco_qk_norm_rope(_p(out), heads * dim, dim, _p(x), heads * dim, dim, _p(w), _p(cos),
                              _p(sin), tokens, heads, dim, rotary_dim, max(seq_len, 1), pos_offset,
                              eps)
    return out


def gated_rms(x: np.ndarray, z: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """``((x*s)*w)*silu(z)`` per ``[tokens, heads, width]`` row (z un-activated)."""
    x, z, w = _f32(x), _f32(z), _f32(w)
    tokens, heads, width = x.shape
    out = np.empty_like(x)
    _load().qdco_gated_rms(_p(out), heads * width, _p(x), heads * width, _p(z), heads * width, _p(w),
                           tokens, heads, width, eps)
    return out


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """``silu(gate) * up`` elementwise on ``[tokens, width]``."""
    gate, up = _f32(gate), _f32(up)
    width = gate.shape[-1]
    tokens = gate.size // width if width else 0
    out = np.empty_like(gate)
    _load().qdco_swiglu(_p(out), width, _p(gate), width, _p(up), width, tokens, width)
    return out


def silu(x: np.ndarray) -> np.ndarray:
    """``native_silu`` (``src/backbone.jl:196-197``) in fp32 numpy."""
    x = _f32(x)
    with np.errstate(over="ignore"):
        return x * (np.float32(1) / (np.float32(1) + np.exp(-x)))
