"""Device operators of the fused row kernels, on PyTorch-ROCm tensors.

Names and argument meanings follow the reference's operator interface for this
path (the generic functions the AMDGPU extension overrides):

==========================  ====================================================
``native_gather``           ``src/backbone.jl:55``; AMDGPU ``ext/amdgpu_workspace.jl:219-236``
``native_rms``              ``src/backbone.jl:200-204``; AMDGPU ``ext/amdgpu_workspace.jl:130-149``
``native_residual_rms``     ``src/backbone.jl:347-350``; AMDGPU ``ext/amdgpu_workspace.jl:157-166``
``prepare_heads``           q/k norm + RoPE of ``full_attention`` (``src/backbone.jl:226-235``;
                            AMDGPU ``prepare_head_kernel!`` ``ext/amdgpu_attention.jl:1-43``)
``native_gated_rms``        ``src/backbone.jl:339-341``; AMDGPU ``ext/amdgpu_delta.jl:181-184``
``native_mlp_gate``         ``native_mlp_gate!`` ``src/backbone.jl:352-355``; AMDGPU
                            ``mlp_gate_kernel!`` ``ext/amdgpu_mlp.jl:63-75``
==========================  ====================================================

Tensors are row-major ``[rows, width]`` (the reference's column-major
``(width, rows)``).  The producers of GEMM inputs (the norms, SwiGLU and the
attention gate merge) also write the split two-term bf16 form, ``out_dtype=BF16X2``:
each fp32 result ``v`` as ``hi = bf16(v)`` and ``lo = bf16(v - hi)``, every aligned
group of 4 elements a 16-byte piece ``[4 hi | 4 lo]``, so a ``[rows, K]`` result
is a bf16 tensor ``[rows, 2K]``; :func:`split_weight` repeats a GEMM weight's rows
in the same pattern and :func:`join_split` reads ``hi + lo`` back.  Every call enqueues one kernel of ``libqdc_hip.so`` on the
tensor device's current PyTorch stream; torch supplies device memory and the
stream only.  dtype is float32 or bfloat16 (fp32 arithmetic either way).
Argument errors raise ``ValueError`` before anything is enqueued, as the
reference raises ``ArgumentError`` / ``DimensionMismatch``: every tensor a call
reads or writes, caller-supplied outputs included, must be on the device of the
call's first input and of the dtype the kernel writes there.
"""
from __future__ import annotations

from typing import Sequence

import numpy as np
import torch

from . import _lib
from ._lib import check, lib

_DTYPES = {torch.float32: _lib.QDC_F32, torch.bfloat16: _lib.QDC_BF16}
BF16X2 = "bf16x2"  # out_dtype of the split two-term bf16 form


def _is_split(out_dtype) -> bool:
    if isinstance(out_dtype, str):
        if out_dtype != BF16X2:
            raise ValueError(f"unknown out_dtype {out_dtype!r}; expected a torch dtype or BF16X2")
        return True
    return False


def _split_stride(stride: int) -> int:
    """A split output's row stride in bf16 values -> in split elements (two bf16
    terms each); rows must start on a whole 16-byte piece (8 bf16 values)."""
    if stride % 8:
        raise ValueError("a split output's rows must be a multiple of 8 bf16 values apart")
    return stride // 2


def split_weight(weight: torch.Tensor) -> torch.Tensor:
    """A GEMM weight ``[K, N]`` (``y = x @ weight``) as ``[2K, N]`` for split
    inputs: rows ``8g + j`` and ``8g + 4 + j`` both hold row ``4g + j``, so
    ``x2 @ split_weight(w)`` = ``(hi + lo) @ w`` for the split form ``x2`` of ``x``."""
    K, N = weight.shape
    if K % 4:
        raise ValueError("the split form needs a multiple of 4 input rows")
    return weight.reshape(K // 4, 1, 4, N).expand(K // 4, 2, 4, N).reshape(2 * K, N).contiguous()


def join_split(x: torch.Tensor) -> torch.Tensor:
    """fp32 ``hi + lo`` of a split tensor (bf16, last axis ``2K``) -> ``[..., K]``."""
    if x.dtype != torch.bfloat16 or x.shape[-1] % 8:
        raise ValueError("a split tensor is bf16 with a last axis of whole 8-value pieces")
    g = x.reshape(*x.shape[:-1], x.shape[-1] // 8, 2, 4).float()
    return (g[..., 0, :] + g[..., 1, :]).reshape(*x.shape[:-1], x.shape[-1] // 2)


def _dtype_code(*tensors) -> int:
    dt = tensors[0].dtype
    for t in tensors:
        if t.dtype != dt:
            raise ValueError(f"dtype mismatch: {dt} vs {t.dtype}")
    if dt not in _DTYPES:
        raise ValueError(f"unsupported dtype {dt}; expected float32 or bfloat16")
    return _DTYPES[dt]


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _device(*tensors) -> None:
    dev = tensors[0].device
    if dev.type != "cuda":
        raise ValueError("device tensors required (torch.device('cuda'))")
    for t in tensors:
        if t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")


def _vector(t: torch.Tensor, n: int, name: str) -> None:
    """A parameter vector the kernel reads as ``n`` contiguous elements."""
    if t.numel() != n or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous vector of {n} elements")


def _rope_tables(tables, rotary_dim: int, like: torch.Tensor):
    """``(cos, sin)`` fp32 ``[n_pos, rotary_dim // 2]`` contiguous device tables
    (``(None, None)`` without rotation); ``n_pos`` is checked against the
    positions by the library."""
    if not rotary_dim:
        return None, None
    if tables is None or len(tables) != 2:
        raise ValueError("rotation needs the (cos, sin) tables of rope_tables")
    cos, sin = tables
    _device(like, cos, sin)
    for t in (cos, sin):
        if (t.dtype != torch.float32 or t.dim() != 2 or t.shape != cos.shape
                or t.shape[1] != rotary_dim // 2 or not t.is_contiguous()):
            raise ValueError("cos and sin must be contiguous float32 [n_pos, rotary_dim//2] "
                             "tables of one shape")
    return cos, sin


def _rows_view(x: torch.Tensor):
    """(rows, width, row_stride) of a tensor whose rows are its last axis,
    contiguous within a row and evenly strided between rows."""
    if x.dim() == 0:
        raise ValueError("expected at least one dimension")
    width = x.shape[-1]
    if x.numel() == 0:
        return 0, width, max(width, 1)
    if x.dim() == 1:
        return 1, width, width
    if width > 1 and x.stride(-1) != 1:
        raise ValueError("rows must be contiguous in their last axis")
    flat = x.reshape(-1, width) if not x.is_contiguous() else x.view(-1, width)
    if flat.data_ptr() != x.data_ptr():
        raise ValueError("rows must be evenly strided (a view, not a copy)")
    return flat.shape[0], width, flat.stride(0) if flat.shape[0] > 1 else width


# ------------------------------------------------------------------ gather --
def native_gather(embedding: torch.Tensor, ids, out: torch.Tensor | None = None,
                  out_dtype: torch.dtype | None = None,
                  error_flag: torch.Tensor | None = None) -> torch.Tensor:
    """``hidden[t, :] = embedding[ids[t], :]`` (0-based ids), bit-exact.

    ``embedding`` is the ``[vocab, hidden]`` table.  Host ids (a sequence or numpy
    array) are range-checked first (``src/backbone.jl:417-418``) and uploaded as
    int32, as the reference AMDGPU path does; a device int32 tensor is used as is
    (then an out-of-range id writes a zero row and sets ``error_flag``)."""
    _device(embedding)
    vocab, hidden = embedding.shape
    if isinstance(ids, torch.Tensor) and ids.device.type != "cpu":
        if ids.dtype != torch.int32 or not ids.is_contiguous():
            raise ValueError("device ids must be a contiguous int32 tensor")
        dev_ids = ids
    else:
        host = np.ascontiguousarray(np.asarray(ids, dtype=np.int64).reshape(-1))
        check(lib().qdc_check_ids(host.ctypes.data, host.size, vocab), "native_gather")
        dev_ids = torch.from_numpy(host.astype(np.int32)).to(embedding.device, non_blocking=False)
    n = dev_ids.numel()
    out_dtype = out_dtype or embedding.dtype
    if out is None:
        out = torch.empty((n, hidden), dtype=out_dtype, device=embedding.device)
    _device(embedding, dev_ids, out)
    if out.shape != (n, hidden) or not out.is_contiguous() or out.dtype != out_dtype:
        raise ValueError("out must be a contiguous [n_ids, hidden] tensor of out_dtype")
    if out_dtype not in _DTYPES:
        raise ValueError("out_dtype must be float32 or bfloat16")
    if not embedding.is_contiguous():
        raise ValueError("embedding must be contiguous")
    flag = 0
    if error_flag is not None:
        _device(embedding, error_flag)
        if error_flag.dtype != torch.int32 or error_flag.numel() < 1:
            raise ValueError("error_flag must be an int32 device tensor")
        flag = error_flag.data_ptr()
    check(lib().qdc_embedding_gather(out.data_ptr(), _DTYPES[out_dtype], embedding.data_ptr(),
                                     _dtype_code(embedding), dev_ids.data_ptr(), n, vocab, hidden,
                                     flag, _stream(embedding)), "native_gather")
    return out


def native_gather_rms(embedding: torch.Tensor, ids: torch.Tensor, weight: torch.Tensor,
                      eps: float, token_mask: torch.Tensor | None = None,
                      error_flag: torch.Tensor | None = None, hidden: torch.Tensor | None = None,
                      normed: torch.Tensor | None = None, normed_dtype=None):
    """The gather fused with the first layer's input norm: returns ``(hidden,
    normed)``, ``hidden [n, width]`` fp32 = the gathered rows (the residual
    stream) and ``normed`` = their zero-centred RMSNorm in the weight's dtype
    (or, with ``normed_dtype=BF16X2`` and a bf16 weight, the split form
    ``[n, 2*width]``), times ``token_mask`` when given.  ``ids`` a contiguous
    device int32 vector; an id outside the vocabulary gives zero rows and sets
    ``error_flag``."""
    _device(embedding, ids, weight)
    if ids.dtype != torch.int32 or not ids.is_contiguous() or ids.dim() != 1:
        raise ValueError("ids must be a contiguous int32 device vector")
    if embedding.dim() != 2 or not embedding.is_contiguous() or embedding.dtype not in _DTYPES:
        raise ValueError("embedding must be a contiguous float32/bfloat16 [vocab, width] tensor")
    vocab, width = embedding.shape
    if weight.dtype not in _DTYPES or weight.numel() != width or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous float32/bfloat16 vector of the row width")
    n = ids.numel()
    split = _is_split(normed_dtype)
    if split and weight.dtype != torch.bfloat16:
        raise ValueError("the split output takes a bfloat16 weight")
    nshape = (n, 2 * width) if split else (n, width)
    if hidden is None:
        hidden = torch.empty((n, width), dtype=torch.float32, device=embedding.device)
    if normed is None:
        normed = torch.empty(nshape, dtype=weight.dtype, device=embedding.device)
    _device(embedding, hidden, normed)
    if (hidden.dtype != torch.float32 or hidden.shape != (n, width)
            or not hidden.is_contiguous()):
        raise ValueError("hidden must be a contiguous float32 [n_ids, width] tensor")
    if normed.dtype != weight.dtype or normed.shape != nshape or not normed.is_contiguous():
        raise ValueError("normed must be a contiguous [n_ids, width] tensor of the weight's dtype "
                         "([n_ids, 2*width] bfloat16 for the split form)")
    keep = _row_mask(token_mask, n, embedding)
    flag = 0
    if error_flag is not None:
        _device(embedding, error_flag)
        if error_flag.dtype != torch.int32 or error_flag.numel() < 1:
            raise ValueError("error_flag must be an int32 device tensor")
        flag = error_flag.data_ptr()
    check(lib().qdc_embedding_gather_rmsnorm(hidden.data_ptr(), normed.data_ptr(),
                                             embedding.data_ptr(), _DTYPES[embedding.dtype],
                                             ids.data_ptr(), weight.data_ptr(),
                                             _lib.QDC_BF16X2 if split else _DTYPES[weight.dtype],
                                             0 if keep is None else keep.data_ptr(), n, vocab,
                                             width, eps, flag, _stream(embedding)),
          "native_gather_rms")
    return hidden, normed


# ------------------------------------------------------------------ norms ---
def _row_mask(token_mask: torch.Tensor | None, rows: int, like: torch.Tensor):
    """Validate an optional device int32 row mask (one 0/1 entry per row)."""
    if token_mask is None:
        return None
    _device(like, token_mask)
    if (token_mask.dtype != torch.int32 or not token_mask.is_contiguous()
            or token_mask.numel() != rows):
        raise ValueError("token_mask must be a contiguous int32 vector of one entry per row")
    return token_mask


def native_rms(x: torch.Tensor, weight: torch.Tensor, eps: float, centered: bool = True,
               out: torch.Tensor | None = None,
               token_mask: torch.Tensor | None = None, out_dtype=None) -> torch.Tensor:
    """RMSNorm over the last axis: ``(x*s)*(1+w)`` (centred) or ``(x*s)*w``.

    The output takes the weight's dtype, so an fp32 ``x`` with a bf16 weight
    gives a bf16 result (an fp32 residual stream feeding bf16 GEMMs);
    ``out_dtype=BF16X2`` (fp32 ``x``, bf16 weight) writes the split form, a
    bf16 tensor with a last axis of ``2*width``.  With a
    ``token_mask`` (device int32, one 0/1 entry per row) each output row is
    multiplied by its entry before rounding: the DeltaNet input mask of
    ``src/backbone.jl:286`` fused into the norm that produces that input."""
    _device(x, weight)
    if x.dtype not in _DTYPES or weight.dtype not in _DTYPES:
        raise ValueError("x and weight must be float32 or bfloat16")
    rows, width, ld_x = _rows_view(x)
    if weight.numel() != width or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous vector of the row width")
    split = _is_split(out_dtype)
    if split and (x.dtype != torch.float32 or weight.dtype != torch.bfloat16):
        raise ValueError("the split output takes float32 rows and a bfloat16 weight")
    oshape = x.shape[:-1] + (2 * width,) if split else x.shape
    if out is None:
        out = torch.empty(oshape, dtype=weight.dtype, device=x.device)
    _device(x, out)
    if out.shape != oshape or out.dtype != weight.dtype:
        raise ValueError("out must have the shape of x and the dtype of weight (the split "
                         "form: bfloat16, last axis 2*width)")
    _, _, ld_out = _rows_view(out)
    if split:
        ld_out = _split_stride(ld_out)  # the C ABI counts split elements
    code = _lib.QDC_BF16X2 if split else _DTYPES[weight.dtype]
    keep = _row_mask(token_mask, rows, x)
    if keep is None:
        check(lib().qdc_rmsnorm(out.data_ptr(), x.data_ptr(), weight.data_ptr(), rows, width,
                                ld_x, ld_out, eps, int(bool(centered)), _DTYPES[x.dtype],
                                code, _stream(x)), "native_rms")
    else:
        check(lib().qdc_rmsnorm_masked(out.data_ptr(), x.data_ptr(), weight.data_ptr(),
                                       keep.data_ptr(), rows, width, ld_x, ld_out, eps,
                                       int(bool(centered)), _DTYPES[x.dtype],
                                       code, _stream(x)), "native_rms")
    return out


def native_residual_rms(x: torch.Tensor, mixed: torch.Tensor, weight: torch.Tensor, eps: float,
                        residual: torch.Tensor | None = None,
                        out: torch.Tensor | None = None,
                        token_mask: torch.Tensor | None = None, out_dtype=None):
    """``residual = x + mixed``; returns ``(residual, rms(residual))`` in one pass.

    ``residual`` has x's dtype, the normalised output the weight's dtype;
    ``mixed`` may be bf16 while x is fp32 (fp32 residual stream).
    ``out_dtype=BF16X2`` (fp32 ``x`` and ``mixed``, bf16 weight) writes the
    normalised rows in the split form (last axis ``2*width``).  A
    ``token_mask`` masks the normalised rows as in ``native_rms``; the residual
    is never masked."""
    _device(x, mixed, weight)
    for t in (x, mixed, weight):
        if t.dtype not in _DTYPES:
            raise ValueError("tensors must be float32 or bfloat16")
    if x.shape != mixed.shape or not x.is_contiguous() or not mixed.is_contiguous():
        raise ValueError("x and mixed must be contiguous tensors of one shape")
    width = x.shape[-1]
    rows = x.numel() // width if width else 0
    _vector(weight, width, "weight")
    split = _is_split(out_dtype)
    if split and (x.dtype != torch.float32 or mixed.dtype != torch.float32
                  or weight.dtype != torch.bfloat16):
        raise ValueError("the split output takes float32 x and mixed and a bfloat16 weight")
    oshape = x.shape[:-1] + (2 * width,) if split else x.shape
    residual = torch.empty_like(x) if residual is None else residual
    out = torch.empty(oshape, dtype=weight.dtype, device=x.device) if out is None else out
    _device(x, residual, out)
    if residual.shape != x.shape or not residual.is_contiguous() or residual.dtype != x.dtype:
        raise ValueError("residual must be a contiguous tensor like x")
    if out.shape != oshape or not out.is_contiguous() or out.dtype != weight.dtype:
        raise ValueError("out must be contiguous, shaped like x, of the weight's dtype (the "
                         "split form: bfloat16, last axis 2*width)")
    code = _lib.QDC_BF16X2 if split else _DTYPES[weight.dtype]
    keep = _row_mask(token_mask, rows, x)
    if keep is None:
        check(lib().qdc_residual_rmsnorm(residual.data_ptr(), out.data_ptr(), x.data_ptr(),
                                         mixed.data_ptr(), weight.data_ptr(), rows, width, eps,
                                         _DTYPES[x.dtype], _DTYPES[mixed.dtype], code,
                                         _stream(x)), "native_residual_rms")
    else:
        check(lib().qdc_residual_rmsnorm_masked(residual.data_ptr(), out.data_ptr(), x.data_ptr(),
                                                mixed.data_ptr(), weight.data_ptr(),
                                                keep.data_ptr(), rows, width, eps,
                                                _DTYPES[x.dtype], _DTYPES[mixed.dtype], code,
                                                _stream(x)),
              "native_residual_rms")
    return residual, out


def native_gated_rms(x: torch.Tensor, z: torch.Tensor, weight: torch.Tensor, eps: float,
                     out: torch.Tensor | None = None, out_dtype=None) -> torch.Tensor:
    """``((x*s)*w)*silu(z)`` per ``[tokens, heads, width]`` row, not centred.

    ``z`` may be a strided view (heads contiguous inside each token), e.g. the
    z block of a packed projection.  ``out_dtype=BF16X2`` (bf16 ``x``, ``z`` and
    weight) writes the split form ``[tokens, heads, 2*width]``."""
    _device(x, z, weight)
    code = _dtype_code(x, z, weight)
    if x.dim() != 3 or z.shape != x.shape:
        raise ValueError("x and z must be [tokens, heads, width]")
    tokens, heads, width = x.shape
    _vector(weight, width, "weight")
    for t in (x, z):
        if t.stride(2) != 1 or (heads > 1 and t.stride(1) != width):
            raise ValueError("heads must be contiguous within a token")
    split = _is_split(out_dtype)
    if split and x.dtype != torch.bfloat16:
        raise ValueError("the split output takes bfloat16 x, z and weight")
    ow = 2 * width if split else width
    if out is None:
        out = torch.empty((tokens, heads, ow), dtype=x.dtype, device=x.device)
    _device(x, out)
    if out.dtype != x.dtype:
        raise ValueError(f"out must have the dtype of x ({x.dtype}), got {out.dtype}")
    if out.shape != (tokens, heads, ow) or out.stride(2) != 1 or (
            heads > 1 and out.stride(1) != ow):
        raise ValueError("out must be [tokens, heads, width] with contiguous heads "
                         "([tokens, heads, 2*width] for the split form)")
    tok = lambda t: t.stride(0) if tokens > 1 else heads * t.shape[2]  # noqa: E731
    out_tok = _split_stride(tok(out)) if split else tok(out)  # the C ABI counts split elements
    check(lib().qdc_gated_rmsnorm(out.data_ptr(), x.data_ptr(), z.data_ptr(), weight.data_ptr(),
                                  tokens, heads, width, tok(x), tok(z), out_tok, eps, code,
                                  _lib.QDC_BF16X2 if split else code, _stream(x)),
          "native_gated_rms")
    return out


# ------------------------------------------------------------------- RoPE ---
def rope_tables(n_pos: int, rotary_dim: int, theta: float, device) -> tuple:
    """fp32 ``[n_pos, rotary_dim//2]`` cos/sin tables built on the host the way
    the reference CPU path builds them (``src/backbone_cpu.jl:90-111``), then
    copied to ``device``."""
    half = rotary_dim // 2
    cos = np.empty((n_pos, half), np.float32)
    sin = np.empty((n_pos, half), np.float32)
    check(lib().qdc_rope_tables(cos.ctypes.data, sin.ctypes.data, n_pos, rotary_dim, theta),
          "rope_tables")
    return (torch.from_numpy(cos).to(device), torch.from_numpy(sin).to(device))


def prepare_heads(q: torch.Tensor | None, k: torch.Tensor | None, q_norm, k_norm, tables,
                  rotary_dim: int, eps: float, seq_len: int | None = None, pos_offset: int = 0,
                  q_out: torch.Tensor | None = None, k_out: torch.Tensor | None = None):
    """Per-head zero-centred RMSNorm + half-split partial RoPE of Q and K heads.

    ``q`` ``[tokens, heads, head_dim]`` and ``k`` ``[tokens, kv_heads, head_dim]``
    are (possibly strided) views: ``qgate.view(T, H, 2*hd)[:, :, :hd]`` reads q
    straight out of the q||gate projection.  Token ``t`` uses position
    ``pos_offset + t % seq_len``.  ``q_out``/``k_out`` are ``[tokens, heads,
    head_dim]`` views, or ``[batch, seq_len, heads, head_dim]`` views splitting
    the tokens into sequences (``x.permute(0, 2, 1, 3)`` of a ``[batch, heads,
    seq_len, head_dim]`` tensor writes the head-major per-sequence layout of
    batched attention products in the same single launch).  Returns
    ``(q_out, k_out)`` (contiguous ``[tokens, heads, head_dim]`` unless given)."""
    ref = q if q is not None else k
    if ref is None:
        raise ValueError("q or k required")
    tokens, _, head_dim = ref.shape
    seq_len = max(tokens, 1) if seq_len is None else seq_len
    cos, sin = _rope_tables(tables, rotary_dim, ref)
    batched = any(o is not None and o.dim() == 4 for o in (q_out, k_out))

    def side(x, norm, out):
        if x is None:
            return None, None, 0, (0, 0, 0, 0, 0)
        _device(x, norm)
        if x.dim() != 3 or x.shape[0] != tokens or x.shape[2] != head_dim or x.stride(2) != 1:
            raise ValueError("q/k must be [tokens, heads, head_dim] with contiguous rows")
        _vector(norm, head_dim, "q_norm/k_norm")
        if out is None:
            out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
        _device(x, out)
        if out.dtype != x.dtype:
            raise ValueError(f"q_out/k_out must have the dtype of q/k ({x.dtype}), got {out.dtype}")
        if out.dim() == 4:
            n_seq = -(-tokens // seq_len)
            if (out.shape[0] * out.shape[1] != tokens or out.shape[2:] != x.shape[1:]
                    or out.stride(3) != 1 or (n_seq > 1 and out.shape[1] != seq_len)):
                raise ValueError("a 4-D q_out/k_out must be [batch, seq_len, heads, head_dim]")
            seq_stride, tok, head = out.stride(0), out.stride(1), out.stride(2)
        else:
            if out.shape != x.shape or out.stride(2) != 1:
                raise ValueError("q_out/k_out must match q/k")
            tok, head = out.stride(0), out.stride(1)
            seq_stride = seq_len * tok if tokens > seq_len else 0
        return x, out, x.shape[1], (x.stride(0), x.stride(1), seq_stride, tok, head)

    qi, qo, heads, qs = side(q, q_norm, q_out)
    ki, ko, kv_heads, ks = side(k, k_norm, k_out)
    code = _dtype_code(*[t for t in (qi, ki, q_norm if qi is not None else None,
                                     k_norm if ki is not None else None) if t is not None])
    ptr = lambda t: 0 if t is None else t.data_ptr()  # noqa: E731
    head_args = (ptr(qo), ptr(ko), ptr(qi), ptr(ki), ptr(q_norm if qi is not None else None),
                 ptr(k_norm if ki is not None else None),
                 ptr(cos) if rotary_dim else 0, ptr(sin) if rotary_dim else 0,
                 tokens, heads, kv_heads, head_dim, rotary_dim, seq_len,
                 pos_offset, cos.shape[0] if rotary_dim else 0)
    if batched:
        check(lib().qdc_qk_norm_rope_batched(*head_args, *qs, *ks, eps, code, _stream(ref)),
              "prepare_heads")
    else:  # one grid of token rows: the reference-shaped entry point
        flat = lambda s: (s[0], s[1], s[3], s[4])  # noqa: E731
        check(lib().qdc_qk_norm_rope(*head_args, *flat(qs), *flat(ks), eps, code, _stream(ref)),
              "prepare_heads")
    return qo, ko


def attention_prepare(q: torch.Tensor | None, k: torch.Tensor, v: torch.Tensor,
                      q_norm: torch.Tensor | None, k_norm: torch.Tensor, tables, rotary_dim: int,
                      eps: float, batch: int, pos_offset: int = 0, out=None):
    """The attention prologue in one launch (``prepare_head_kernel!`` for Q and K
    and ``prepare_value_kernel!``, ``ext/amdgpu_attention.jl:1-59``): per-head
    zero-centred RMSNorm + half-split partial RoPE of ``q [T, H, hd]`` and
    ``k [T, KV, hd]``, and ``v [T, KV, hd]`` moved, for ``batch`` sequences of
    ``T // batch`` tokens.  ``q``/``k``/``v`` are views with contiguous rows (q may
    stride its heads, e.g. inside a q||gate projection; k and v heads are
    contiguous within a token).  Returns ``(q_out [B, H, S, hd], k_t [B, KV, hd, S],
    v_out [B, KV, S, hd])``: K transposed, so both attention products are plain
    batched GEMMs.  ``out`` optionally supplies the three contiguous outputs.
    ``q=None`` (with ``q_norm=None``) prepares K and V only and returns
    ``(None, k_t, v_out)``: the context of a query projected apart (final-query
    attention)."""
    kv_only = q is None
    if kv_only and q_norm is not None:
        raise ValueError("q_norm without q")
    present = [t for t in (q, k, v, q_norm, k_norm) if t is not None]
    _device(*present)
    code = _dtype_code(*present)
    if (not kv_only and q.dim() != 3) or k.dim() != 3 or v.dim() != 3 or k.shape != v.shape:
        raise ValueError("q must be [T, H, hd] and k, v [T, KV, hd]")
    T, KV, hd = k.shape
    H = 0 if kv_only else q.shape[1]
    if (not kv_only and (q.shape[0] != T or q.shape[2] != hd)) or batch <= 0 or T % batch:
        raise ValueError("q, k and v must share tokens and head_dim; tokens a multiple of batch")
    for t in (q, k, v):
        if t is not None and t.stride(2) != 1:
            raise ValueError("rows must be contiguous")
    for t in (k, v):
        if KV > 1 and t.stride(1) != hd:
            raise ValueError("k and v heads must be contiguous within a token")
    if not kv_only:
        _vector(q_norm, hd, "q_norm")
    _vector(k_norm, hd, "k_norm")
    S = T // batch
    shapes = ((batch, H, S, hd), (batch, KV, hd, S), (batch, KV, S, hd))
    if out is None:
        out = tuple(None if kv_only and i == 0 else
                    torch.empty(sh, dtype=k.dtype, device=k.device) for i, sh in enumerate(shapes))
    if len(out) != 3:
        raise ValueError("out must be three tensors (q, K transposed, v)")
    if kv_only and out[0] is not None:
        raise ValueError("out[0] must be None when q is None")
    for o, sh in zip(out[1:] if kv_only else out, shapes[1:] if kv_only else shapes):
        _device(k, o)
        if o.dtype != k.dtype or tuple(o.shape) != sh or not o.is_contiguous():
            raise ValueError("out must be three contiguous tensors [B, H, S, hd], "
                             "[B, KV, hd, S], [B, KV, S, hd] of k's dtype")
    cos, sin = _rope_tables(tables, rotary_dim, k)
    ptr = lambda t: 0 if t is None else t.data_ptr()  # noqa: E731
    tok = lambda t: t.stride(0) if T > 1 else t.shape[1] * t.shape[2]  # noqa: E731
    check(lib().qdc_attention_prepare(ptr(out[0]), out[1].data_ptr(), out[2].data_ptr(),
                                      ptr(q), k.data_ptr(), v.data_ptr(),
                                      ptr(q_norm), k_norm.data_ptr(), ptr(cos), ptr(sin),
                                      batch, S, H, KV, hd, rotary_dim, pos_offset,
                                      cos.shape[0] if rotary_dim else 0,
                                      0 if kv_only else tok(q),
                                      0 if kv_only else (q.stride(1) if H > 1 else hd),
                                      tok(k), tok(v), eps, code, _stream(k)),
          "attention_prepare")
    return out


# ----------------------------------------------------------------- SwiGLU ---
def native_mlp_gate(gate: torch.Tensor, up: torch.Tensor,
                    out: torch.Tensor | None = None, out_dtype=None) -> torch.Tensor:
    """``silu(gate) * up`` on ``[tokens, width]`` views (contiguous rows).

    ``native_mlp_gate!`` writes into ``gate``; here ``out=gate`` does the same
    (allowed when the strides agree).  For the packed gate||up GEMM output pass
    ``packed[:, :I]`` and ``packed[:, I:]``.  ``out_dtype=BF16X2`` (fp32 gate
    and up) writes the split form ``[tokens, 2*width]``."""
    _device(gate, up)
    code = _dtype_code(gate, up)
    if gate.dim() != 2 or up.shape != gate.shape:
        raise ValueError("gate and up must be [tokens, width]")
    tokens, width = gate.shape
    for t in (gate, up):
        if width > 1 and t.stride(1) != 1:
            raise ValueError("rows must be contiguous")
    split = _is_split(out_dtype)
    if split and gate.dtype != torch.float32:
        raise ValueError("the split output takes float32 gate and up")
    odt, ow = (torch.bfloat16, 2 * width) if split else (gate.dtype, width)
    if out is None:
        out = torch.empty((tokens, ow), dtype=odt, device=gate.device)
    _device(gate, out)
    if out.dtype != odt:
        raise ValueError(f"out must be {odt}, got {out.dtype}")
    if out.shape != (tokens, ow) or (ow > 1 and out.stride(1) != 1):
        raise ValueError("out must be [tokens, width] with contiguous rows "
                         "([tokens, 2*width] bfloat16 for the split form)")
    ld = lambda t: t.stride(0) if tokens > 1 else t.shape[1]  # noqa: E731
    ld_out = _split_stride(ld(out)) if split else ld(out)  # the C ABI counts split elements
    check(lib().qdc_swiglu(out.data_ptr(), gate.data_ptr(), up.data_ptr(), tokens, width,
                           ld(gate), ld(up), ld_out, code, _lib.QDC_BF16X2 if split else code,
                           _stream(gate)), "native_mlp_gate")
    return out


def _token_rows(t: torch.Tensor) -> int | None:
    """Row stride (elements between consecutive tokens) of a ``[B, S, heads, dim]``
    float32 view whose tokens are rows of ``heads * dim`` contiguous elements
    (a contiguous tensor, or a column block of wider rows); None otherwise."""
    B, S, heads, dim = t.shape
    if t.dtype != torch.float32 or t.stride(3) != 1 or (heads > 1 and t.stride(2) != dim):
        return None
    ld = t.stride(1) if S > 1 else (t.stride(0) if B > 1 else heads * dim)
    if ld < heads * dim or (B > 1 and S > 1 and t.stride(0) != S * ld):
        return None
    return ld


def delta_scan(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor,
               decay: torch.Tensor, out_dtype: torch.dtype = torch.float32,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """Gated delta rule recurrence (the DeltaNet "existing path", not a fused
    row op): fp32 q, k ``[B, S, KH, kd]``, v ``[B, S, H, vd]`` whose tokens are
    rows of contiguous heads (contiguous tensors, or the column blocks of one
    ``[T, q|k|v]`` buffer that ``delta_prologue(..., interleaved=True)``
    returns; q and k with the same row stride), contiguous beta and decay
    ``[B, S, H]`` -> ``[B, S, H, vd]`` in ``out_dtype`` (or into ``out``)."""
    _device(q, k, v, beta, decay)
    for t in (beta, decay):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("delta_scan beta and decay must be contiguous float32 tensors")
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k and v must be [B, S, heads, dim]")
    B, S, KH, kd = k.shape
    H, vd = v.shape[2], v.shape[3]
    if q.shape != k.shape or v.shape[:2] != (B, S) or beta.shape != (B, S, H) or \
            decay.shape != (B, S, H):
        raise ValueError("inconsistent delta_scan shapes")
    ld_q, ld_k, ld_v = _token_rows(q), _token_rows(k), _token_rows(v)
    if ld_q is None or ld_k is None or ld_v is None or ld_q != ld_k:
        raise ValueError("q, k and v must be float32 rows of contiguous heads, q and k with "
                         "one row stride")
    if out is None:
        out = torch.empty((B, S, H, vd), dtype=out_dtype, device=q.device)
    _device(q, out)
    if out.shape != (B, S, H, vd) or out.dtype not in _DTYPES or not out.is_contiguous():
        raise ValueError("out must be a contiguous [B, S, H, vd] float32/bfloat16 tensor")
    out_dtype = out.dtype
    check(lib().qdc_delta_scan(out.data_ptr(), _DTYPES[out_dtype], q.data_ptr(), k.data_ptr(),
                               v.data_ptr(), beta.data_ptr(), decay.data_ptr(), B, S, H, KH, kd,
                               vd, ld_k, ld_v, _stream(q)), "delta_scan")
    return out


def delta_prologue(proj: torch.Tensor, conv: torch.Tensor, a_decay: torch.Tensor,
                   dt_bias: torch.Tensor, seq_len: int, key_heads: int, key_dim: int,
                   value_heads: int, value_dim: int, out=None, interleaved: bool = False):
    """DeltaNet prologue on the packed projection ``[T, q|k|v|z|a|b]`` (rows
    contiguous): causal conv + SiLU, q/k L2 norm, beta/decay gates.  Returns fp32
    ``q, k [T, KH, kd]``, ``v [T, H, vd]``, ``beta, decay [T, H]``: contiguous
    tensors, or with ``interleaved`` q, k and v as the column blocks of one
    ``[T, q|k|v]`` buffer (each token's outputs one contiguous row, the layout
    the forward uses; ``delta_scan`` reads it as is).  ``out``: a tuple of five
    tensors of those shapes to write into instead (q, k, v rows of contiguous
    heads, q and k with one row stride; beta and decay contiguous)."""
    _device(proj, conv, a_decay, dt_bias)
    if proj.dtype not in _DTYPES or proj.dim() != 2 or proj.stride(1) != 1:
        raise ValueError("proj must be a [tokens, width] float32/bfloat16 view with unit column stride")
    for t in (conv, a_decay, dt_bias):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError("conv, a_decay and dt_bias must be contiguous float32")
    channels = 2 * key_heads * key_dim + value_heads * value_dim
    if conv.dim() != 2 or conv.shape[0] != channels:
        raise ValueError(f"conv must be [{channels}, taps] (the q|k|v channels)")
    _vector(a_decay, value_heads, "a_decay")
    _vector(dt_bias, value_heads, "dt_bias")
    if proj.shape[1] < channels + value_heads * value_dim + 2 * value_heads:
        raise ValueError("proj rows must hold the q|k|v|z|a|b blocks")
    T = proj.shape[0]
    taps = conv.shape[-1]
    dev = proj.device
    f32 = torch.float32
    shapes = [(T, key_heads, key_dim), (T, key_heads, key_dim), (T, value_heads, value_dim),
              (T, value_heads), (T, value_heads)]
    if out is None:
        if interleaved:
            kw = key_heads * key_dim
            qkv = torch.empty((T, channels), dtype=f32, device=dev)
            out = [qkv[:, :kw].view(shapes[0]), qkv[:, kw:2 * kw].view(shapes[1]),
                   qkv[:, 2 * kw:].view(shapes[2])]
            out += [torch.empty(sh, dtype=f32, device=dev) for sh in shapes[3:]]
        else:
            out = [torch.empty(sh, dtype=f32, device=dev) for sh in shapes]
    elif any(o.dtype != f32 or tuple(o.shape) != sh for o, sh in zip(out, shapes)) or \
            not (out[3].is_contiguous() and out[4].is_contiguous()):
        raise ValueError("out must be five float32 tensors of the output shapes")
    q, k, v, beta, decay = out
    _device(proj, q, k, v, beta, decay)
    rows = [_token_rows(t.unsqueeze(0)) for t in (q, k, v)]
    if None in rows or rows[0] != rows[1]:
        raise ValueError("q, k and v must be rows of contiguous heads, q and k with one row "
                         "stride")
    ld = proj.stride(0) if T > 1 else proj.shape[1]
    check(lib().qdc_delta_prologue(q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(),
                                   decay.data_ptr(), proj.data_ptr(), _DTYPES[proj.dtype], ld,
                                   conv.data_ptr(), taps, a_decay.data_ptr(), dt_bias.data_ptr(), T,
                                   seq_len, key_heads, key_dim, value_heads, value_dim, rows[0],
                                   rows[2], _stream(proj)), "delta_prologue")
    return q, k, v, beta, decay


# ------------------------------------------------------------- attention ---
def attention_softmax(scores: torch.Tensor, mask: torch.Tensor | None, scale: float,
                      q_offset: int = 0, out_dtype=None, out: torch.Tensor | None = None):
    """Masked, scaled softmax of score rows ``[B, H, Q, K]`` (fp32, contiguous):
    query ``q`` sits at position ``q + q_offset``; key ``i`` is visible when
    ``i <= position`` and ``mask[b, i] != 0`` (``mask`` int32 ``[B, K]`` or
    None).  Returns probs ``[B, H, Q, K]`` in ``out_dtype`` (default fp32);
    ``out=scores`` runs in place."""
    _device(scores)
    if scores.dtype != torch.float32 or scores.dim() != 4 or not scores.is_contiguous():
        raise ValueError("scores must be a contiguous float32 [B, H, Q, K] tensor")
    B, H, Q, K = scores.shape
    if mask is not None:
        _device(scores, mask)
        if mask.dtype != torch.int32 or mask.shape != (B, K) or not mask.is_contiguous():
            raise ValueError("mask must be a contiguous int32 [B, K] tensor")
    if out is None:
        out = torch.empty(scores.shape, dtype=out_dtype or torch.float32, device=scores.device)
    _device(scores, out)
    if out.shape != scores.shape or not out.is_contiguous() or out.dtype not in _DTYPES:
        raise ValueError("out must be a contiguous float32/bfloat16 tensor shaped like scores")
    check(lib().qdc_attention_softmax(out.data_ptr(), _DTYPES[out.dtype], scores.data_ptr(),
                                      mask.data_ptr() if mask is not None else 0, B, H, Q, K,
                                      q_offset, float(scale), _stream(scores)),
          "attention_softmax")
    return out


def attention_gate(values: torch.Tensor, gate: torch.Tensor, out_dtype=None,
                   out: torch.Tensor | None = None):
    """Output-gate merge ``out[t, h*hd + r] = values[b, h, s, r] * sigmoid(gate[t, h, r])``
    for ``t = b*S + s``: ``values`` fp32 ``[B, H, S, hd]`` contiguous (the PV
    product), ``gate`` a ``[B*S, H, hd]`` view with unit element stride (the gate
    half of the q||gate projection).  Returns ``[B*S, H*hd]`` in ``out_dtype``
    (default: the gate's), or with ``out_dtype=BF16X2`` the split form
    ``[B*S, 2*H*hd]`` (bf16)."""
    _device(values, gate)
    if values.dtype != torch.float32 or values.dim() != 4 or not values.is_contiguous():
        raise ValueError("values must be a contiguous float32 [B, H, S, hd] tensor")
    B, H, S, hd = values.shape
    if gate.dtype not in _DTYPES or gate.shape != (B * S, H, hd) or gate.stride(2) != 1:
        raise ValueError("gate must be a [B*S, H, hd] view with unit element stride")
    split = _is_split(out_dtype)
    odt = torch.bfloat16 if split else (out_dtype or gate.dtype)
    oshape = (B * S, (2 if split else 1) * H * hd)
    if out is None:
        out = torch.empty(oshape, dtype=odt, device=values.device)
    _device(values, out)
    if (out.dtype not in _DTYPES or (split and out.dtype != odt) or out.shape != oshape
            or out.stride(1) != 1):
        raise ValueError("out must be [B*S, H*hd] with unit element stride "
                         "([B*S, 2*H*hd] bfloat16 for the split form)")
    tok = out.stride(0) if B * S > 1 else oshape[1]
    if split:
        tok = _split_stride(tok)  # the C ABI counts split elements
    gtok = gate.stride(0) if B * S > 1 else H * gate.stride(1)
    code = _lib.QDC_BF16X2 if split else _DTYPES[out.dtype]
    check(lib().qdc_attention_gate(out.data_ptr(), code, values.data_ptr(),
                                   gate.data_ptr(), _DTYPES[gate.dtype], B, S, H, hd, gtok,
                                   gate.stride(1) if H > 1 else hd, tok, _stream(values)),
          "attention_gate")
    return out


def device_copy(dst: torch.Tensor, src: torch.Tensor, chunks_per_thread: int = 1,
                block: int = 256) -> torch.Tensor:
    """Plain copy of ``src``'s bytes into ``dst`` (both contiguous, same byte
    count, a multiple of 16) with the library's streaming copy kernel: the
    single-launch bandwidth ceiling the benchmark sets beside each row kernel.
    ``chunks_per_thread`` (1, 2, 4, 8) and ``block`` (256, 512) select the launch
    shape (``qdc_copy_grid``); the default is ``qdc_copy``'s."""
    _device(dst, src)
    if not dst.is_contiguous() or not src.is_contiguous():
        raise ValueError("dst and src must be contiguous")
    nbytes = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() != nbytes:
        raise ValueError("dst and src must hold the same number of bytes")
    if (chunks_per_thread, block) == (1, 256):
        check(lib().qdc_copy(dst.data_ptr(), src.data_ptr(), nbytes, _stream(src)), "device_copy")
    else:
        check(lib().qdc_copy_grid(dst.data_ptr(), src.data_ptr(), nbytes, chunks_per_thread, block,
                                  _stream(src)), "device_copy")
    return dst


def device_copy_pair(dst0: torch.Tensor, src0: torch.Tensor, dst1: torch.Tensor,
                     src1: torch.Tensor, chunks_per_thread: int = 1, block: int = 256):
    """Two plain copies in one launch (``qdc_copy_pair``): ``src0``'s bytes into
    ``dst0`` and ``src1``'s into ``dst1`` (each pair contiguous, same byte count,
    a multiple of 16), each thread moving its chunks of both: the ceiling the
    benchmark sets beside the row kernels that read two tensors and write two."""
    _device(dst0, src0, dst1, src1)
    counts = []
    for d, s in ((dst0, src0), (dst1, src1)):
        if not d.is_contiguous() or not s.is_contiguous():
            raise ValueError("copy_pair buffers must be contiguous")
        n = s.numel() * s.element_size()
        if d.numel() * d.element_size() != n:
            raise ValueError("each destination must hold its source's byte count")
        counts.append(n)
    check(lib().qdc_copy_pair(dst0.data_ptr(), src0.data_ptr(), counts[0], dst1.data_ptr(),
                              src1.data_ptr(), counts[1], chunks_per_thread, block,
                              _stream(src0)), "device_copy_pair")
    return dst0, dst1


def device_copy_rows(dst: torch.Tensor, table: torch.Tensor, rows: torch.Tensor,
                     repeat: int = 1) -> torch.Tensor:
    """``dst[i]`` = ``repeat`` copies of the bytes of ``table[rows[i]]`` (``table``
    ``[n, width]`` contiguous, ``rows`` device int32, ``dst`` contiguous with
    ``repeat`` times a table row's bytes per row): the gather's access pattern
    with no conversion, the ceiling the benchmark sets beside the gathers."""
    _device(table, rows, dst)
    if not dst.is_contiguous() or not table.is_contiguous() or table.dim() != 2:
        raise ValueError("table must be a contiguous 2-D tensor and dst contiguous")
    if rows.dtype != torch.int32 or not rows.is_contiguous():
        raise ValueError("rows must be a contiguous int32 tensor")
    row_bytes = table.shape[1] * table.element_size()
    if dst.numel() * dst.element_size() != rows.numel() * row_bytes * repeat:
        raise ValueError("dst must hold repeat copies of one table row per index")
    check(lib().qdc_copy_rows(dst.data_ptr(), table.data_ptr(), rows.data_ptr(), rows.numel(),
                              table.shape[0], row_bytes, repeat, _stream(table)),
          "device_copy_rows")
    return dst


def empty_launch(workgroups: int, device) -> None:
    """A launch of ``workgroups`` workgroups that do nothing on ``device``'s
    current stream: the fixed cost of a grid of that size."""
    check(lib().qdc_empty(workgroups, torch.cuda.current_stream(device).cuda_stream),
          "empty_launch")


def check_ids(ids: Sequence[int], vocab: int) -> None:
    """Host id check of ``check_sequence`` (``src/backbone.jl:417-418``)."""
    host = np.ascontiguousarray(np.asarray(ids, dtype=np.int64).reshape(-1))
    status = lib().qdc_check_ids(host.ctypes.data, host.size, vocab)
    if status == -4:
        raise ValueError("Token ID is outside the vocabulary.")
    check(status, "check_ids")
