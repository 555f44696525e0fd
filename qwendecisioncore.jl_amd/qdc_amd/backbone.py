"""``backbone_hidden`` on MI355X with the fused row kernels.

Mirrors the reference's public entry points and their validation:

* :class:`QwenBackbone` -- ``QwenBackbone(dir; device=:amdgpu)`` (``src/backbone.jl:74-192``):
  weights uploaded once, projection weights stored transposed and packed
  (``[qkv; z; a; b]`` and ``[gate; up]`` the way the reference's AMDGPU extension
  packs them, ``ext/amdgpu_mlp.jl:15-52``; the attention projections as
  ``[q; k; v; gate]``, q_proj's per-head q and gate rows regrouped).
* :func:`backbone_hidden` / :func:`backbone_last_hidden` (``src/backbone.jl:433-501``):
  one sequence per call, ids checked on the host (``check_sequence`` :413-422).
* :func:`batch_backbone_hidden`: the optional batched hook (``src/backbone.jl:66-70``),
  one final-normalised last-position state per row; :func:`batch_backbone_states`
  returns every position of every row.

Per layer (``native_layer``, ``src/backbone.jl:363-388``) the fused kernels do
the row work: the embedding gather is fused with the first input RMSNorm, each
later layer's input RMSNorm with the previous layer's MLP
residual add (``qdc_residual_rmsnorm``; the last one with the final norm) and,
before a DeltaNet layer, with its input mask (``qdc_residual_rmsnorm_masked``),
post-attention residual + RMSNorm, the attention prologue (q/k norm + partial
RoPE, and K transposed and V head-major for the two products, read straight out
of the packed projection), the attention masked softmax and output-gate merge, the
DeltaNet prologue (convolution, SiLU, q/k L2 norm, gates), the gated-delta
recurrence, the DeltaNet gated RMSNorm reading z inside the packed projection,
and SwiGLU reading the packed gate||up GEMM output.  GEMMs and the two attention
products run through PyTorch-ROCm (hipBLASLt), with fp32 results; attention
scores and probabilities are fp32 (probabilities stored in the model dtype for
the PV product).

``split_gemm_inputs=True`` (or ``"all"``; bf16 models) stores every GEMM input
-- the normalised rows, the SwiGLU output, the merged attention output and the
gated norm output -- in the split two-term bf16 form written by the kernels
that produce them (``ops.BF16X2``), against projection weights whose input rows
are repeated in the same pattern (``ops.split_weight``): the GEMMs stay bf16 x
bf16 with fp32 accumulation and twice the inner dimension, while their inputs
keep about 16 significant bits.  The MLP gate/up projection then writes fp32
for SwiGLU; the attention and DeltaNet projections, q/k, the probabilities and
the recurrence output stay bf16.  ``split_gemm_inputs="mlp"`` splits only the
two MLP inputs (the post-attention norm and the SwiGLU output), where bf16
rounding is amplified most, and leaves the other GEMMs at their bf16 size.
"""
from __future__ import annotations

import os

import numpy as np
import torch

from . import ops
from .config import BackboneConfig, load_config
from .weights import read_checkpoint_tensors



class QwenBackbone:
    """A Qwen3.5 hybrid backbone resident on one GPU."""

    def __init__(self, cfg: BackboneConfig, weights: dict, device="cuda:0",
                 dtype: torch.dtype = torch.float32, split_gemm_inputs: bool | str = False):
        """``dtype`` is the storage type of weights and GEMM activations; the
        residual stream and the returned hidden states are fp32 either way.
        ``split_gemm_inputs`` (bfloat16 only: False, True / ``"all"``, or
        ``"mlp"``) selects the split GEMM inputs described in the module
        docstring."""
        if dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("dtype must be float32 or bfloat16")
        modes = {False: None, None: None, "none": None, True: "all", "all": "all", "mlp": "mlp"}
        if split_gemm_inputs not in modes:
            raise ValueError("split_gemm_inputs must be False, True, 'all' or 'mlp'")
        self.split = modes[split_gemm_inputs]
        if self.split and dtype != torch.bfloat16:
            raise ValueError("split GEMM inputs are a bfloat16 mode")
        self.cfg, self.dtype = cfg, dtype
        # a split row holds whole groups of 4 elements
        widths = {"mlp": (cfg.hidden, cfg.intermediate),
                  "all": (cfg.hidden, cfg.intermediate, cfg.head_dim, cfg.value_dim)}
        if self.split and any(w % 4 for w in widths[self.split]):
            raise ValueError(f"split GEMM inputs ({self.split!r}) need the widths "
                             f"{widths[self.split]} to be multiples of 4")
        # out_dtype of the kernels that write GEMM inputs: the MLP's two inputs,
        # and every other GEMM input
        self.mlp_in = ops.BF16X2 if self.split else None
        self.gemm_in = ops.BF16X2 if self.split == "all" else None
        self.device = torch.device(device)
        self._tables = {}

        def dev(x, dt=None):
            t = x if isinstance(x, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(x))
            return t.to(self.device).to(dt or dtype).contiguous()

        def gemm_weight(w, split):  # [out, in] -> [in, out] (input rows repeated when split)
            w = w.t().contiguous()
            return ops.split_weight(w) if split else w

        def lin(*names, pad_to=1, mlp=False):  # packed, transposed [in, out] for y = x @ W
            w = torch.cat([dev(weights[n]) for n in names], 0)
            extra = -w.shape[0] % pad_to
            if extra:  # zero output columns: the GEMM runs a tile-aligned width
                w = torch.cat([w, w.new_zeros((extra, w.shape[1]))], 0)
            return gemm_weight(w, self.mlp_in if mlp else self.gemm_in)

        self.embedding = dev(weights["embed_tokens.weight"])
        # the last residual add is fused with the final norm, which writes fp32
        self.final_norm = dev(weights["norm.weight"], torch.float32)
        self.layers = []
        for i, kind in enumerate(cfg.layer_types):
            p = f"layers.{i}."
            layer = {
                "kind": kind,
                "input_norm": dev(weights[p + "input_layernorm.weight"]),
                "post_norm": dev(weights[p + "post_attention_layernorm.weight"]),
                "gate_up": lin(p + "mlp.gate_proj.weight", p + "mlp.up_proj.weight", mlp=True),
                "down": lin(p + "mlp.down_proj.weight", mlp=True),
            }
            if kind == "full_attention":
                a = p + "self_attn."
                # q_proj's rows are [q_h; gate_h] per head; regrouped so the packed
                # projection of a token is [q (all heads) | k | v | gate (all heads)]:
                # the attention prologue reads q, k and v as one contiguous span
                # and the gate merge reads the gate block whole
                hd, H = cfg.head_dim, cfg.heads
                qg = dev(weights[a + "q_proj.weight"]).reshape(H, 2, hd, -1)
                layer.update(qkv=gemm_weight(torch.cat([qg[:, 0].reshape(H * hd, -1),
                                                        dev(weights[a + "k_proj.weight"]),
                                                        dev(weights[a + "v_proj.weight"]),
                                                        qg[:, 1].reshape(H * hd, -1)], 0),
                                             self.gemm_in),
                             out=lin(a + "o_proj.weight"), q_norm=dev(weights[a + "q_norm.weight"]),
                             k_norm=dev(weights[a + "k_norm.weight"]))
            elif kind == "linear_attention":
                a = p + "linear_attn."
                conv = weights[a + "conv1d.weight"]
                conv = conv if isinstance(conv, torch.Tensor) else torch.from_numpy(np.asarray(conv))
                a_log = weights[a + "A_log"]
                a_log = a_log if isinstance(a_log, torch.Tensor) else torch.from_numpy(np.asarray(a_log))
                layer.update(
                    # [qkv | z | a | b] is 2 value-head columns past a multiple of 256
                    # at the Qwen3.5 shapes; padding the packed width to 256 lets
                    # hipBLASLt use its full tiles (measured 354 -> 282 us at 16384
                    # tokens x 1024 -> 8224 vs 8448 columns)
                    proj=lin(a + "in_proj_qkv.weight", a + "in_proj_z.weight",
                             a + "in_proj_a.weight", a + "in_proj_b.weight", pad_to=256),
                    conv=dev(conv.reshape(conv.shape[0], conv.shape[-1]), torch.float32),
                    # fixed decay multiplier, computed once in fp32 (src/backbone.jl:160-162)
                    a_decay=(-1.0 * torch.exp(a_log.to(torch.float32))).to(self.device).contiguous(),
                    dt_bias=dev(weights[a + "dt_bias"], torch.float32),
                    norm=dev(weights[a + "norm.weight"]),
                    out=lin(a + "out_proj.weight"))
            else:
                raise ValueError(f"Unsupported layer type {kind}.")
            self.layers.append(layer)

    @classmethod
    def from_weights(cls, weights: dict, cfg: BackboneConfig, device="cuda:0",
                     dtype: torch.dtype = torch.float32,
                     split_gemm_inputs: bool | str = False) -> "QwenBackbone":
        return cls(cfg, weights, device, dtype, split_gemm_inputs)

    @classmethod
    def from_directory(cls, directory: str, device="cuda:0",
                       dtype: torch.dtype = torch.float32,
                       split_gemm_inputs: bool | str = False) -> "QwenBackbone":
        """A local safetensors checkpoint directory (no network access).  Tensors
        load straight onto ``device`` in their stored dtype; with ``dtype=bfloat16``
        a BF16 checkpoint is never widened to fp32 (the packed projection weights
        are assembled on the device in bf16)."""
        cfg = load_config(directory)
        weights = read_checkpoint_tensors(directory, device=device)
        cfg = BackboneConfig(**{**cfg.as_dict(), "vocab": weights["embed_tokens.weight"].shape[0],
                                "intermediate": weights["layers.0.mlp.gate_proj.weight"].shape[0],
                                "layer_types": cfg.layer_types})
        return cls(cfg, weights, device, dtype, split_gemm_inputs)

    def _mm(self, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        """A projection whose result feeds a row kernel, in the model dtype."""
        return a @ b

    def _mm32(self, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        """A GEMM whose result feeds the fp32 residual stream: fp32 output even
        from bf16 operands (hipBLASLt accumulates in fp32 either way)."""
        if a.dtype == torch.float32:
            return a @ b
        return torch.mm(a, b, out_dtype=torch.float32)

    @property
    def vocab(self) -> int:
        return self.embedding.shape[0]

    def rope_tables(self, seq_len: int):
        key = seq_len
        if key not in self._tables:
            self._tables[key] = ops.rope_tables(seq_len, self.cfg.rotary_dim, self.cfg.rope_theta,
                                                self.device)
        return self._tables[key]

    # ------------------------------------------------------------ forward --
    @torch.no_grad()
    def forward(self, ids: torch.Tensor, mask: torch.Tensor | None, last_only: bool = False,
                error_flag: torch.Tensor | None = None) -> torch.Tensor:
        """Final-normalised hidden states ``[B*S, hidden]`` (device, fp32)
        for device ids ``[B, S]`` (int32) and mask ``[B, S]`` (0/1); ``mask=None``
        means every token is kept (no masking work is done).

        ``last_only`` returns ``[B, hidden]``, the last position of each row:
        a full-attention last layer attends from each row's last query only
        (:meth:`_final_query_attention`), and after the last attention block only
        those rows go through the last MLP and the final norm (the last-token
        forward ``native_hidden_forward``, ``src/backbone.jl:390-396``).  ``error_flag`` (device int32, cleared by
        the caller) is set by the gather when an id is outside the vocabulary."""
        B, S = ids.shape
        cfg = self.cfg
        mask32 = None if mask is None else mask.to(torch.int32).contiguous()
        # Masked tokens are zeroed before the DeltaNet projections (src/backbone.jl:286):
        # the norm producing a DeltaNet layer's input writes the masked rows itself.
        keep = None if mask32 is None else mask32.view(-1)
        delta_keep = lambda i: keep if self.layers[i]["kind"] != "full_attention" else None  # noqa: E731
        # the gather fused with the first input norm: the residual stream h in
        # fp32 (a bf16 table widens exactly) and its normalised rows in one pass
        h, normed = ops.native_gather_rms(self.embedding, ids.reshape(-1).contiguous(),
                                          self.layers[0]["input_norm"], cfg.eps,
                                          token_mask=delta_keep(0), error_flag=error_flag,
                                          normed_dtype=self.gemm_in)
        for i, layer in enumerate(self.layers):
            last = i + 1 == len(self.layers)
            # the last-token forward's last attention layer attends from the
            # last query only (its attention output comes back as [B, hidden])
            final_query = last and last_only and layer["kind"] == "full_attention"
            if final_query:
                mixed = self._final_query_attention(layer, normed, mask32, B, S)
            elif layer["kind"] == "full_attention":
                mixed = self._full_attention(layer, normed, mask32, B, S)
            else:
                mixed = self._delta_attention(layer, normed, B, S)
            if last and last_only:  # the MLP and the final norm of the last rows only
                h = h.view(B, S, -1)[:, -1].contiguous()
                if not final_query:
                    mixed = mixed.view(B, S, -1)[:, -1].contiguous()
            residual, normed = ops.native_residual_rms(h, mixed, layer["post_norm"], cfg.eps,
                                                       out_dtype=self.mlp_in)
            # split inputs: fp32 gate/up for SwiGLU (bf16 there costs ~6x the
            # end-to-end error of the whole split pipeline)
            gate_up = (self._mm32 if self.split else self._mm)(normed, layer["gate_up"])
            inter = gate_up.shape[1] // 2
            act = ops.native_mlp_gate(gate_up[:, :inter], gate_up[:, inter:],
                                      out_dtype=self.mlp_in)
            down = self._mm32(act, layer["down"])
            nxt = self.final_norm if last else self.layers[i + 1]["input_norm"]
            # residual add of the MLP fused with the next RMSNorm
            h, normed = ops.native_residual_rms(residual, down, nxt, cfg.eps,
                                                token_mask=None if last else delta_keep(i + 1),
                                                out_dtype=None if last else self.gemm_in)
        return normed

    def _full_attention(self, layer, x, mask32, B, S):
        """``full_attention`` in the AMDGPU form (``ext/amdgpu_attention.jl:108-178``;
        generic ``src/backbone.jl:224-262``).  One prologue launch normalises and
        rotates q and k and moves v out of the packed projection into the layouts
        the products read: q ``[B, H, S, hd]``, K transposed ``[B, KV, hd, S]``,
        v ``[B, KV, S, hd]``.  The G = H / KV query heads sharing a KV head are one
        ``[G*S, hd]`` block, so both products are plain batched GEMMs over
        (sequence, KV head), with no K/V expansion and no layout copy.  The
        masked softmax and the gate merge are HIP kernels."""
        cfg = self.cfg
        hd, H, KV = cfg.head_dim, cfg.heads, cfg.kv_heads
        G = H // KV
        T = B * S
        proj = self._mm(x, layer["qkv"])                     # [T, q | k | v | gate]
        q_in = proj[:, :H * hd].view(T, H, hd)
        k_in = proj[:, H * hd:(H + KV) * hd].view(T, KV, hd)
        v_in = proj[:, (H + KV) * hd:(H + 2 * KV) * hd].view(T, KV, hd)
        gate = proj[:, (H + 2 * KV) * hd:].view(T, H, hd)
        tables = self.rope_tables(S) if cfg.rotary_dim else None
        q, kt, v = ops.attention_prepare(q_in, k_in, v_in, layer["q_norm"], layer["k_norm"],
                                         tables, cfg.rotary_dim, cfg.eps, B)
        scores = self._bmm32(q.view(B * KV, G * S, hd), kt.view(B * KV, hd, S))  # [B*KV, G*S, S]
        scale = float(np.float32(1) / np.sqrt(np.float32(hd)))      # inv(sqrt(Float32(dim)))
        probs = ops.attention_softmax(scores.view(B, H, S, S), mask32, scale, out_dtype=self.dtype,
                                      out=scores.view(B, H, S, S) if self.dtype == torch.float32
                                      else None)
        values = self._bmm32(probs.view(B * KV, G * S, S), v.view(B * KV, S, hd))  # [B, H, S, hd]
        merged = ops.attention_gate(values.view(B, H, S, hd), gate,
                                    out_dtype=self.gemm_in or self.dtype)
        return self._mm32(merged, layer["out"])

    def _final_query_attention(self, layer, x, mask32, B, S):
        """Final-query attention of the last-token forward: K and V over the
        whole context, q and its gate for each sequence's last position only, as
        the reference's CPU and CUDA last-token paths do
        (``cpu_final_full_attention``, ``src/backbone_cpu.jl:984-1034``, chosen at
        ``:1106-1131``; ``full_attention_last``, ``ext/cuda_attention.jl:188-267``).
        The query keeps its position S - 1 (rotated there, ``:1026-1034``) and
        sees every kept key.  Returns the attention output of the last rows,
        ``[B, hidden]`` fp32: the S x S scores, softmax and PV work of the full
        form shrink to one query row per head."""
        cfg = self.cfg
        hd, H, KV = cfg.head_dim, cfg.heads, cfg.kv_heads
        G = H // KV
        T = B * S
        w = layer["qkv"]                                     # [in, q | k | v | gate]
        kv = self._mm(x, w[:, H * hd:(H + 2 * KV) * hd])    # [T, k | v] of every token
        proj = self._mm(x.view(B, S, -1)[:, -1], w)          # [B, q | k | v | gate], last rows
        tables = self.rope_tables(S) if cfg.rotary_dim else None
        _, kt, v = ops.attention_prepare(None, kv[:, :KV * hd].view(T, KV, hd),
                                         kv[:, KV * hd:].view(T, KV, hd), None, layer["k_norm"],
                                         tables, cfg.rotary_dim, cfg.eps, B)
        # q norm + RoPE of the B last rows, each at position S - 1
        q, _ = ops.prepare_heads(proj[:, :H * hd].view(B, H, hd), None, layer["q_norm"], None,
                                 tables, cfg.rotary_dim, cfg.eps, seq_len=1, pos_offset=S - 1)
        scores = self._bmm32(q.view(B * KV, G, hd), kt.view(B * KV, hd, S))      # [B*KV, G, S]
        scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
        probs = ops.attention_softmax(scores.view(B, H, 1, S), mask32, scale, q_offset=S - 1,
                                      out_dtype=self.dtype,
                                      out=scores.view(B, H, 1, S) if self.dtype == torch.float32
                                      else None)
        values = self._bmm32(probs.view(B * KV, G, S), v.view(B * KV, S, hd))  # [B, H, 1, hd]
        gate = proj[:, (H + 2 * KV) * hd:].view(B, H, hd)
        merged = ops.attention_gate(values.view(B, H, 1, hd), gate,
                                    out_dtype=self.gemm_in or self.dtype)
        return self._mm32(merged, layer["out"])

    def _bmm32(self, a, b):
        """Batched product with an fp32 result (fp32 accumulate for bf16 inputs)."""
        if a.dtype == torch.float32:
            return torch.bmm(a, b)
        return torch.bmm(a, b, out_dtype=torch.float32)

    def _delta_attention(self, layer, x, B, S):
        """Gated DeltaNet (``src/backbone.jl:284-345``; recurrent form
        ``src/backbone_cpu.jl:680-759``) on an input whose masked tokens the
        producing norm has already zeroed (``native_layer_outputs(...,
        Val(true))``, ``src/backbone.jl:372-376``)."""
        cfg = self.cfg
        kd, kh, vd, vh = cfg.key_dim, cfg.key_heads, cfg.value_dim, cfg.value_heads
        T = B * S
        kw, vw = kd * kh, vd * vh
        cq = 2 * kw + vw
        proj = self._mm(x, layer["proj"])  # [T, cq + vw + 2*vh (+ zero padding)]
        # conv + SiLU, q/k L2 norm and the beta/decay gates in one pass; q, k, v
        # are the column blocks of one [T, q|k|v] buffer (one output row per token)
        q, k, v, beta, decay = ops.delta_prologue(proj, layer["conv"], layer["a_decay"],
                                                  layer["dt_bias"], S, kh, kd, vh, vd,
                                                  interleaved=True)
        q, k = q.view(B, S, kh, kd), k.view(B, S, kh, kd)
        v, beta, decay = v.view(B, S, vh, vd), beta.view(B, S, vh), decay.view(B, S, vh)
        # recurrence straight into the model dtype the gated norm reads
        result = ops.delta_scan(q, k, v, beta, decay, self.dtype)
        z = proj[:, cq:cq + vw].view(T, vh, vd)
        out = ops.native_gated_rms(result.view(T, vh, vd), z, layer["norm"], cfg.eps,
                                   out_dtype=self.gemm_in)
        return self._mm32(out.view(T, -1), layer["out"])


# ---------------------------------------------------------------- API -------
def check_sequence(model: QwenBackbone, ids, mask) -> None:
    """``check_sequence`` (``src/backbone.jl:413-422``), ValueError for ArgumentError."""
    ids = np.asarray(ids)
    mask = np.asarray(mask)
    if ids.size != mask.size:
        raise ValueError("Input IDs and mask must have identical lengths.")
    if ids.size == 0:
        raise ValueError("Inputs must not be empty.")
    ops.check_ids(ids, model.vocab)
    if not np.isin(mask, (0, 1)).all():
        raise ValueError("Mask values must be zero or one.")


def _host_sequence(model, ids, mask):
    """One sequence's ids and mask as checked 1-D int64 host arrays (a ``[1, S]``
    array is taken as its row)."""
    ids = np.asarray(ids, dtype=np.int64)
    mask = np.asarray(mask, dtype=np.int64)
    if ids.ndim == 2:
        if ids.shape[0] != 1 or mask.shape[0] != 1:
            raise ValueError("Pass one sequence per call; batching is not implemented yet.")
        ids, mask = ids[0], mask[0]
    check_sequence(model, ids, mask)
    return ids.reshape(-1), mask.reshape(-1)


def _device_inputs(model, ids, mask):
    ids, mask = _host_sequence(model, ids, mask)
    d_ids = torch.from_numpy(ids.astype(np.int32)).to(model.device).view(1, -1)
    if mask.all():  # nothing masked: the forward skips the masking work
        return d_ids, None
    d_mask = torch.from_numpy(mask.astype(np.int32)).to(model.device).view(1, -1)
    return d_ids, d_mask


def backbone_hidden(model: QwenBackbone, ids, mask, positions=None) -> np.ndarray:
    """Final-normalised hidden states ``[len(ids), hidden]`` (fp32, host) of one
    sequence; ``positions`` (1-based) selects rows as the reference does."""
    d_ids, d_mask = _device_inputs(model, ids, mask)
    states = model.forward(d_ids, d_mask).float().cpu().numpy()
    if positions is None:
        return states
    positions = np.asarray(positions, dtype=np.int64)
    if positions.size and (positions.min() < 1 or positions.max() > states.shape[0]):
        raise ValueError("Position is outside the sequence.")
    return states[positions - 1]


def backbone_last_hidden(model: QwenBackbone, ids, mask) -> np.ndarray:
    """Final-normalised hidden state of the last position, a ``[hidden]`` vector
    (``src/backbone.jl:470-490``): the last-token forward, which normalises and
    copies back only that row."""
    d_ids, d_mask = _device_inputs(model, ids, mask)
    return model.forward(d_ids, d_mask, last_only=True)[0].float().cpu().numpy()


def native_sequence_start(mask, row: int) -> int:
    """0-based index of row ``row``'s first kept token: the leading masked
    tokens are skipped unless ``QDC_AMDGPU_TRIM_PADDING`` is set to something
    other than ``"1"`` (then 0), and the last token always stays
    (``native_sequence_start``, ``ext/QwenDecisionCoreAMDGPUExt.jl:17-24``).
    Leading masked tokens leave the kept tokens' states unchanged up to
    rounding: they are zero DeltaNet inputs and masked attention keys, and
    rotary attention scores depend only on relative positions."""
    if os.environ.get("QDC_AMDGPU_TRIM_PADDING", "1") != "1":
        return 0
    row_mask = np.asarray(mask)[row]
    start = 0
    while start < row_mask.shape[0] - 1 and row_mask[start] == 0:
        start += 1
    return start


def _batch_inputs(model: QwenBackbone, ids, mask, trim: bool = False):
    """``[B, S]`` ids and mask as device tensors, checked as ``check_sequence``
    checks one sequence (``src/backbone.jl:413-422``).  Host inputs are checked
    before anything runs.  Device ids are checked by the gather itself (an id
    outside the vocabulary sets a device flag) and a device mask by a device
    comparison; both are read after the forward by :func:`_raise_if_invalid`.
    Returns ``(ids, mask or None, pending)``."""
    if not isinstance(ids, torch.Tensor) or ids.device.type != "cuda":
        ids = np.asarray(ids, dtype=np.int64)
        host_mask = np.ones(ids.shape, np.int64) if mask is None else np.asarray(mask, np.int64)
        if ids.ndim != 2 or host_mask.shape != ids.shape:
            raise ValueError("Input IDs and mask must be [batch, sequence] arrays of one shape.")
        check_sequence(model, ids.reshape(-1), host_mask.reshape(-1))
        if trim:  # from the earliest first kept token of the rows
            # (ext/metal_batch_forward.jl:113-116, 124-125)
            first = min(native_sequence_start(host_mask, r) for r in range(ids.shape[0]))
            ids, host_mask = ids[:, first:], host_mask[:, first:]
        d_ids = torch.from_numpy(ids.astype(np.int32)).to(model.device)
        d_mask = None if host_mask.all() else torch.from_numpy(
            host_mask.astype(np.int32)).to(model.device)
        return d_ids, d_mask, None
    if ids.dim() != 2 or ids.numel() == 0:
        raise ValueError("Inputs must be a non-empty [batch, sequence] array.")
    if ids.dtype not in (torch.int32, torch.int64):
        raise ValueError("Token IDs must be integers.")
    if ids.dtype == torch.int64:  # ids beyond int32 cannot be in the vocabulary
        ids = torch.clamp(ids, -1, model.vocab).to(torch.int32)
    flag = torch.zeros(1, dtype=torch.int32, device=model.device)
    bad_mask = None
    if mask is not None:
        if not isinstance(mask, torch.Tensor) or mask.device != ids.device:
            raise ValueError("A device id tensor needs its mask on the same device.")
        if mask.shape != ids.shape:
            raise ValueError("Input IDs and mask must have identical lengths.")
        bad_mask = ((mask != 0) & (mask != 1)).any()
        mask = mask.to(torch.int32)
    return ids.contiguous(), mask, (flag, bad_mask)


def _raise_if_invalid(pending) -> None:
    if pending is None:
        return
    flag, bad_mask = pending
    if int(flag.item()) != 0:
        raise ValueError("Token ID is outside the vocabulary.")
    if bad_mask is not None and bool(bad_mask.item()):
        raise ValueError("Mask values must be zero or one.")


def batch_backbone_hidden(model: QwenBackbone, ids, mask) -> np.ndarray:
    """The optional batched hook (``batch_backbone_hidden``, ``src/backbone.jl:66-70``;
    Metal ``ext/metal_batch_forward.jl:100-138``): ``B`` equal-length sequences,
    ids and 0/1 mask ``[B, S]`` (host arrays, or device tensors; ``mask=None``:
    nothing masked) -> the final-normalised hidden state of each row's last
    position, ``[B, hidden]`` fp32 on the host (the reference's
    ``(hidden, batch)``).  RoPE positions restart at 0 for every row.  With host
    inputs the masked columns before every row's first kept token are dropped
    first (:func:`native_sequence_start`), as the reference's batched hook does.
    Invalid ids or mask values raise ``ValueError`` as ``check_sequence`` does."""
    d_ids, d_mask, pending = _batch_inputs(model, ids, mask, trim=True)
    flag = None if pending is None else pending[0]
    out = model.forward(d_ids, d_mask, last_only=True, error_flag=flag)
    _raise_if_invalid(pending)
    return out.float().cpu().numpy()


def batch_backbone_states(model: QwenBackbone, ids, mask) -> torch.Tensor:
    """Every position of ``B`` equal-length sequences: as :func:`batch_backbone_hidden`
    but returning all final-normalised states ``[B, S, hidden]`` (fp32) on the
    device, the batched form of ``backbone_hidden``."""
    d_ids, d_mask, pending = _batch_inputs(model, ids, mask)
    flag = None if pending is None else pending[0]
    B, S = d_ids.shape
    out = model.forward(d_ids, d_mask, error_flag=flag).view(B, S, -1)
    _raise_if_invalid(pending)
    return out
