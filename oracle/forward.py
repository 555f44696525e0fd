"""CPU restatement of ``backbone_hidden`` for end-to-end parity checks.

TEST INFRASTRUCTURE ONLY (see ``qdc_oracle.py``).  The in-scope row ops go
through the C oracle; the GEMMs, attention and the DeltaNet recurrence are
numpy fp32 restatements of the reference's generic and CPU paths.

Weights are a dict of float32 numpy arrays keyed by the checkpoint names with
the ``language_model.`` prefix removed (``layers.0.mlp.gate_proj.weight`` ...),
laid out as stored (PyTorch ``[out, in]``), which is the reference's Julia
``(in, out)`` matrix in the same memory.

``bf16=True`` (``storage="bf16"``) runs the same algorithm with bf16 storage (RNE,
``src/safetensors.jl:37-42``) of the activations a bf16 device pipeline keeps in
bf16: the normalised GEMM inputs, the outputs of the input-side projections
(q||gate, k, v, qkv, z, a, b, gate, up), the normed+rotated q/k, the attention
probabilities, the merged attention output, the DeltaNet recurrence and gated-norm outputs and the SwiGLU
output.  The residual stream and the outputs of the residual-side projections
(o_proj, out_proj, down_proj) stay fp32.  Arithmetic stays fp32 throughout.

``storage="bf16x2"`` is the split-GEMM-input pipeline: every GEMM input (the
normalised rows, the merged attention output, the gated-norm output and the
SwiGLU output) is stored as two bf16 terms (``qdc_oracle.round_split``), the MLP
gate/up projections stay fp32, and the attention and DeltaNet projections, the
normed+rotated q/k, the probabilities and the recurrence output are bf16.
``storage="bf16x2_mlp"`` splits only the two MLP inputs (the post-attention
norm and the SwiGLU output); the other GEMM inputs are bf16.
"""
from __future__ import annotations

import numpy as np

from . import qdc_oracle as ops

F32 = np.float32
FLOATMAX = np.finfo(np.float32).max


def config_from_text_config(cfg: dict) -> dict:
    """Config parsing of ``QwenBackbone`` (``src/backbone.jl:84-106``)."""
    if cfg.get("attention_bias", False):
        raise ValueError("Attention biases are not supported.")
    if cfg.get("hidden_act", "silu") != "silu":
        raise ValueError("Expected SiLU activation.")
    rope = cfg["rope_parameters"]
    if rope.get("rope_type", "default") != "default":
        raise ValueError("Only default RoPE is supported.")
    out = dict(
        hidden=int(cfg["hidden_size"]),
        head_dim=int(cfg["head_dim"]),
        heads=int(cfg["num_attention_heads"]),
        kv_heads=int(cfg["num_key_value_heads"]),
        key_heads=int(cfg["linear_num_key_heads"]),
        value_heads=int(cfg["linear_num_value_heads"]),
        key_dim=int(cfg["linear_key_head_dim"]),
        value_dim=int(cfg["linear_value_head_dim"]),
        eps=float(F32(cfg["rms_norm_eps"])),
        rope_theta=float(F32(rope["rope_theta"])),
        # only rope_parameters.partial_rotary_factor is read (src/backbone.jl:101)
        rotary_dim=int(cfg["head_dim"] * rope.get("partial_rotary_factor", 1.0)),
        layer_types=list(cfg["layer_types"]),
    )
    if out["value_heads"] % out["key_heads"]:
        raise ValueError("Value heads must be a multiple of key heads.")
    if out["heads"] % out["kv_heads"]:
        raise ValueError("Query heads must be a multiple of KV heads.")
    return out


def _silu(x):
    return ops.silu(x)


def _sigmoid(x):
    x = x.astype(F32)
    with np.errstate(over="ignore"):
        return F32(1) / (F32(1) + np.exp(-x))


def _softplus(x):
    """``native_softplus`` (``src/backbone.jl:198``)."""
    x = x.astype(F32)
    return np.maximum(x, F32(0)) + np.log1p(np.exp(-np.abs(x))).astype(F32)


def _linear(x, w):
    """``native_linear``: y[T, out] = x[T, in] @ W[out, in]^T in fp32."""
    return (x @ w.T).astype(F32)


STORAGE = ("f32", "bf16", "bf16x2", "bf16x2_mlp")


def _storage(bf16, storage) -> str:
    st = storage or ("bf16" if bf16 else "f32")
    if st not in STORAGE:
        raise ValueError(f"storage must be one of {STORAGE}")
    return st


def _store(x, st, role="act"):
    """Storage rounding of an activation of ``role`` under storage policy ``st``:
    ``mlp_in`` (an MLP GEMM input), ``gemm_in`` (another GEMM input), ``mlp_proj``
    (the MLP gate/up projections) or ``act`` (any other stored activation)."""
    split = st.startswith("bf16x2")
    if st == "f32" or (split and role == "mlp_proj"):
        return np.asarray(x, F32)
    if (split and role == "mlp_in") or (st == "bf16x2" and role == "gemm_in"):
        return ops.round_split(x)
    return ops.round_bf16(x)


def full_attention(W: dict, p: str, x: np.ndarray, mask: np.ndarray, cfg: dict, tables,
                   bf16: bool = False, trace: dict | None = None, storage: str | None = None):
    """``full_attention`` (``src/backbone.jl:224-262``) on ``x [T, hidden]``.

    ``trace``, when given, receives the intermediates under the names of the
    stages (``qgate``, ``k_proj``, ``v``, ``q``, ``k``, ``scores``, ``probs``,
    ``values``, ``merged``, ``mixed``), each as stored."""
    st = _storage(bf16, storage)
    T = x.shape[0]
    hd, H, KV = cfg["head_dim"], cfg["heads"], cfg["kv_heads"]
    qgate = _store(_linear(x, W[p + "self_attn.q_proj.weight"]), st).reshape(T, H, 2 * hd)
    cos, sin = tables
    q = _store(ops.qk_norm_rope(qgate[:, :, :hd], W[p + "self_attn.q_norm.weight"], cos, sin,
                                cfg["rotary_dim"], cfg["eps"]), st)
    kp = _store(_linear(x, W[p + "self_attn.k_proj.weight"]), st).reshape(T, KV, hd)
    k = _store(ops.qk_norm_rope(kp, W[p + "self_attn.k_norm.weight"], cos, sin, cfg["rotary_dim"],
                                cfg["eps"]), st)
    v = _store(_linear(x, W[p + "self_attn.v_proj.weight"]), st).reshape(T, KV, hd)
    # AMDGPU form (ext/amdgpu_attention.jl:148-176): scores of every head, the
    # masked softmax with scale inv(sqrt(dim)), the PV product, the gate merge;
    # kv head of query head h is h // (H // KV) (src/backbone.jl:249-251)
    groups = H // KV
    qh = q.transpose(1, 0, 2)                                   # [H, T, hd]
    kh = np.repeat(k.transpose(1, 0, 2), groups, axis=0)        # [H, T, hd]
    vh = np.repeat(v.transpose(1, 0, 2), groups, axis=0)
    scores = (qh @ kh.transpose(0, 2, 1)).astype(F32)           # [H, query, key]
    probs = _store(attention_softmax(scores[None], mask[None], F32(1) / np.sqrt(F32(hd)))[0],
                   st)
    values = (probs @ vh).astype(F32)                           # [H, query, hd]
    merged = _store(attention_gate(values[None], qgate[:, :, hd:]), st, "gemm_in")
    mixed = _linear(merged, W[p + "self_attn.o_proj.weight"])
    if trace is not None:
        trace.update(qgate=qgate, k_proj=kp, v=v, q=q, k=k, scores=scores, probs=probs,
                     values=values, merged=merged, mixed=mixed)
    return mixed


def attention_softmax(scores: np.ndarray, mask, scale, q_offset: int = 0) -> np.ndarray:
    """``attention_softmax_kernel!`` (``ext/amdgpu_attention.jl:61-88``) on score
    rows ``[B, H, Q, K]``: query q sits at position ``q + q_offset``; key i is
    visible when ``i <= position`` and ``mask[b, i] == 1`` (``mask`` ``[B, K]`` or
    None); value = ``scores * scale`` if visible else ``-floatmax``; then
    ``exp(value - max) / sum``.  A row with no visible key is uniform over all K
    keys, as in the reference."""
    B, H, Q, K = scores.shape
    pos = np.arange(Q)[:, None] + q_offset
    vis = np.broadcast_to(np.arange(K)[None, :] <= pos, (B, Q, K))
    if mask is not None:
        vis = vis & (np.asarray(mask)[:, None, :] != 0)
    value = np.where(vis[:, None], scores.astype(F32) * F32(scale), F32(-FLOATMAX)).astype(F32)
    with np.errstate(over="ignore", invalid="ignore"):
        e = np.exp(value - value.max(axis=-1, keepdims=True)).astype(F32)
    return (e / e.sum(axis=-1, keepdims=True)).astype(F32)


def attention_gate(values: np.ndarray, gate: np.ndarray) -> np.ndarray:
    """``merge_gate_kernel!`` (``ext/amdgpu_attention.jl:90-106``): values
    ``[B, H, S, hd]`` times ``sigmoid(gate)`` for gate ``[B*S, H, hd]``, written
    as ``[B*S, H*hd]``."""
    B, H, S, hd = values.shape
    merged = values.transpose(0, 2, 1, 3).reshape(B * S, H, hd) * _sigmoid(gate)
    return merged.reshape(B * S, H * hd).astype(F32)


def causal_depthwise(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """``causal_depthwise`` (``src/backbone.jl:264-276``): x [T, C], w [C, K], then SiLU."""
    T, C = x.shape
    K = w.shape[1]
    out = np.zeros((T, C), F32)
    for index in range(K):
        lag = K - 1 - index
        if lag >= T:
            continue
        out[lag:, :] += x[:T - lag, :] * w[:, index][None, :]
    return _silu(out)


def delta_attention(W: dict, p: str, x: np.ndarray, mask: np.ndarray, cfg: dict,
                    bf16: bool = False, trace: dict | None = None, storage: str | None = None):
    """Gated DeltaNet, recurrent form of the CPU default path.

    ``cpu_delta_prepare`` (``src/backbone_cpu.jl:465-499``) and
    ``cpu_delta_recurrent_heads!`` / ``cpu_delta_recurrent_step!``
    (``src/backbone_cpu.jl:680-759``), which equals the chunked generic form
    ``delta_attention`` (``src/backbone.jl:284-345``) up to rounding.
    ``trace``, when given, receives the intermediates (``masked``, ``qkv``,
    ``z``, ``a``, ``b``, ``q``, ``k``, ``v``, ``beta``, ``decay``,
    ``recurrence`` (fp32), ``result`` (stored), ``gated``, ``mixed``)."""
    st = _storage(bf16, storage)
    T = x.shape[0]
    kd, kh, vd, vh = cfg["key_dim"], cfg["key_heads"], cfg["value_dim"], cfg["value_heads"]
    masked = (x * mask.astype(F32)[:, None]).astype(F32)
    qkv = _store(_linear(masked, W[p + "linear_attn.in_proj_qkv.weight"]), st)
    conv = W[p + "linear_attn.conv1d.weight"]
    conv = conv.reshape(conv.shape[0], conv.shape[-1])
    z = _store(_linear(masked, W[p + "linear_attn.in_proj_z.weight"]), st).reshape(T, vh, vd)
    b_raw = _store(_linear(masked, W[p + "linear_attn.in_proj_b.weight"]), st)
    a_raw = _store(_linear(masked, W[p + "linear_attn.in_proj_a.weight"]), st)
    a_decay = (F32(-1) * np.exp(W[p + "linear_attn.A_log"].astype(F32))).astype(F32)
    q, k, v, beta, decay = delta_prologue(qkv, conv, a_raw, b_raw, a_decay,
                                          W[p + "linear_attn.dt_bias"], kh, kd, vh, vd)
    recurrence = delta_recurrence(q, k, v, beta, decay)
    result = _store(recurrence, st)
    out = _store(ops.gated_rms(result, z, W[p + "linear_attn.norm.weight"], cfg["eps"]), st,
                 "gemm_in")
    mixed = _linear(out.reshape(T, vh * vd), W[p + "linear_attn.out_proj.weight"])
    if trace is not None:
        trace.update(masked=masked, qkv=qkv, z=z, a=a_raw, b=b_raw, q=q, k=k, v=v, beta=beta,
                     decay=decay, recurrence=recurrence, result=result, gated=out, mixed=mixed)
    return mixed


def normalize_heads(x, multiplier):
    """L2-normalise the last axis, ``x * inv(sqrt(sum(x^2) + 1e-6) * multiplier)``
    in fp32: the loop form of ``cpu_normalize_delta_heads!``
    (``src/backbone_cpu.jl:411-427``), also the AMDGPU ``qk_normalize_kernel!``
    scale (``ext/amdgpu_delta.jl:1-33``)."""
    x = np.asarray(x, dtype=F32)
    with np.errstate(over="ignore", invalid="ignore"):
        squared = (x * x).sum(-1, keepdims=True, dtype=F32)
        return (x * (F32(1) / (np.sqrt(squared + F32(1e-6)) * F32(multiplier)))).astype(F32)


def delta_prologue(qkv, conv, a_raw, b_raw, a_decay, dt_bias, kh, kd, vh, vd):
    """Causal conv + SiLU of the qkv projection, q/k L2 normalisation and the
    gates, for one sequence (``cpu_delta_prepare``, ``src/backbone_cpu.jl:465-499``;
    generic ``src/backbone.jl:286-296``; ``cpu_normalize_delta_heads!`` :411-427
    with its scale-then-multiply form).  Returns q, k ``[T, kh, kd]``, v
    ``[T, vh, vd]``, beta, decay ``[T, vh]``, all fp32."""
    T = qkv.shape[0]
    mixed = causal_depthwise(qkv, conv)
    kw = kd * kh
    q = mixed[:, :kw].reshape(T, kh, kd)
    k = mixed[:, kw:2 * kw].reshape(T, kh, kd)
    v = mixed[:, 2 * kw:].reshape(T, vh, vd)
    q = normalize_heads(q, np.sqrt(F32(kd)))
    k = normalize_heads(k, F32(1))
    beta = _sigmoid(b_raw)
    decay = (a_decay * _softplus(a_raw + dt_bias)).astype(F32)
    return q, k, np.ascontiguousarray(v), beta, decay


def delta_recurrence(q, k, v, beta, decay):
    """Gated delta rule, token by token, for one sequence:
    ``cpu_delta_recurrent_step!`` (``src/backbone_cpu.jl:681-705``) inside
    ``cpu_delta_recurrent_heads!`` (:710-759).  q, k ``[T, KH, kd]``, v
    ``[T, H, vd]``, beta and decay ``[T, H]`` -> ``[T, H, vd]`` fp32; value
    head h reads key head ``h // (H // KH)`` (``cld(head, groups)``, 1-based)."""
    T, H, vd = v.shape
    kh, kd = k.shape[1], k.shape[2]
    kidx = np.arange(H) // (H // kh)
    state = np.zeros((H, vd, kd), F32)
    result = np.empty((T, H, vd), F32)
    for t in range(T):
        factor = np.exp(decay[t]).astype(F32)                     # [H]
        kt = k[t, kidx]                                            # [H, kd]
        qt = q[t, kidx]
        proj = np.einsum("hvk,hk->hv", state, kt).astype(F32)
        proj = (beta[t][:, None] * (v[t] - factor[:, None] * proj)).astype(F32)
        state = (factor[:, None, None] * state + proj[:, :, None] * kt[:, None, :]).astype(F32)
        result[t] = np.einsum("hvk,hk->hv", state, qt)
    return result


def check_sequence(ids, mask, vocab):
    """``check_sequence`` (``src/backbone.jl:413-422``)."""
    ids = np.asarray(ids)
    mask = np.asarray(mask)
    if ids.size != mask.size:
        raise ValueError("Input IDs and mask must have identical lengths.")
    if ids.size == 0:
        raise ValueError("Inputs must not be empty.")
    if ids.min() < 0 or ids.max() >= vocab:
        raise ValueError("Token ID is outside the vocabulary.")
    if not np.isin(mask, (0, 1)).all():
        raise ValueError("Mask values must be zero or one.")


def backbone_layer(W: dict, cfg: dict, i: int, h: np.ndarray, normed: np.ndarray,
                   mask: np.ndarray, tables, bf16: bool = False, trace: dict | None = None,
                   storage: str | None = None):
    """Layer ``i`` of ``native_hidden_states`` (``native_layer``,
    ``src/backbone.jl:358-388``) from the residual stream ``h`` and its input
    norm ``normed``: returns the next ``(h, normed)``, where ``normed`` is the next
    layer's input norm (the final norm after the last layer) fused with the MLP
    residual add.  ``trace`` also receives ``residual``, ``post_normed``, ``gate``,
    ``up``, ``act`` and ``down`` besides the attention intermediates."""
    st = _storage(bf16, storage)
    eps = cfg["eps"]
    kinds = cfg["layer_types"]
    p = f"layers.{i}."
    if kinds[i] == "full_attention":
        mixed = full_attention(W, p, normed, mask, cfg, tables, trace=trace, storage=st)
    elif kinds[i] == "linear_attention":
        mixed = delta_attention(W, p, normed, mask, cfg, trace=trace, storage=st)
    else:
        raise ValueError(f"Unsupported layer type {kinds[i]}.")
    residual, post = ops.residual_rms(h, mixed, W[p + "post_attention_layernorm.weight"], eps)
    post = _store(post, st, "mlp_in")
    gate = _store(_linear(post, W[p + "mlp.gate_proj.weight"]), st, "mlp_proj")
    up = _store(_linear(post, W[p + "mlp.up_proj.weight"]), st, "mlp_proj")
    act = _store(ops.swiglu(gate, up), st, "mlp_in")
    down = _linear(act, W[p + "mlp.down_proj.weight"])
    last = i + 1 == len(kinds)
    nxt = W["norm.weight"] if last else W[f"layers.{i + 1}.input_layernorm.weight"]
    # native_residual_add! (src/backbone.jl:358-361), then the next RMSNorm
    h, normed = ops.residual_rms(residual, down, nxt, eps)
    if not last:
        normed = _store(normed, st, "gemm_in")
    if trace is not None:
        trace.update(residual=residual, post_normed=post, gate=gate, up=up, act=act, down=down)
    return h, normed


def embed(W: dict, cfg: dict, ids, mask, bf16: bool = False, storage: str | None = None):
    """Checked ids, the gathered residual stream and the first input norm:
    ``(ids, mask, h, normed, tables)`` (``src/backbone.jl:433-446``)."""
    embed_table = W["embed_tokens.weight"]
    check_sequence(ids, mask, embed_table.shape[0])
    ids = np.asarray(ids, dtype=np.int32).reshape(-1)
    mask = np.asarray(mask, dtype=np.int64).reshape(-1)
    T = ids.size
    h = ops.gather(embed_table, ids)
    tables = ops.rope_tables(T, cfg["rotary_dim"], cfg["rope_theta"]) if cfg["rotary_dim"] else (
        np.zeros((T, 0), F32), np.zeros((T, 0), F32))
    normed = _store(ops.rms(h, W["layers.0.input_layernorm.weight"], cfg["eps"]),
                    _storage(bf16, storage), "gemm_in")
    return ids, mask, h, normed, tables


def backbone_hidden(W: dict, cfg: dict, ids, mask, bf16: bool = False,
                    storage: str | None = None) -> np.ndarray:
    """``backbone_hidden`` (``src/backbone.jl:433-460``) -> ``[T, hidden]`` fp32.

    The residual add of each layer is computed together with the next RMSNorm
    (the final norm after the last layer); ``bf16`` selects bf16 storage of
    the activations listed in the module docstring (``storage`` selects any of
    the policies there)."""
    st = _storage(bf16, storage)
    ids, mask, h, normed, tables = embed(W, cfg, ids, mask, storage=st)
    for i in range(len(cfg["layer_types"])):
        h, normed = backbone_layer(W, cfg, i, h, normed, mask, tables, storage=st)
    return normed
