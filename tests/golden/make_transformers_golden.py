"""Write ``tests/golden/transformers_golden.npz``: expected outputs of the
local ``transformers`` Qwen3.5 modules (an implementation independent of the
reference and of this repository) for the in-scope ops.

Inputs are closed forms (sin/cos ramps, as the reference's own op tests use) or
weights regenerated from a seed by ``qdc_amd.weights.random_weights``, so the
npz stores only the expected outputs plus the few inputs that are not closed
forms.  Offline: nothing is downloaded; models are built from config dicts.

Vectors:
  rms/*      Qwen3_5RMSNorm, x = sin(1..), w = 0.1*cos(1..), widths 7 / 256 / 1024
  gated/*    Qwen3_5RMSNormGated, x = sin, z = 3*cos, w = cos, [17, 4, 128]
  rope/*     Qwen3_5RMSNorm (q_norm/k_norm) + apply_rotary_pos_emb with the
             model's rotary embedding: head_dim 64 / rotary 16 / theta 1e7 and
             head_dim 256 / rotary 64 / theta 1e7 (two sequences, positions reset)
  swiglu/*   ACT2FN["silu"](gate) * up incl. special values
  model/*    Qwen3_5TextModel forward (final-normed hidden states) of the 2-layer
             plumbing backbone (hidden 256, rotary 16 of 64) at 48 tokens, vocab 512
"""
import dataclasses
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "qwendecisioncore.jl_amd"))

from qdc_amd.config import plumbing_config  # noqa: E402
from qdc_amd.weights import random_weights  # noqa: E402

from transformers.models.qwen3_5 import modeling_qwen3_5 as M  # noqa: E402
from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig  # noqa: E402
from transformers.activations import ACT2FN  # noqa: E402

DST = os.path.join(HERE, "transformers_golden.npz")


def ramp(fn, shape, scale=1.0):
    n = int(np.prod(shape))
    return (fn(np.arange(1, n + 1, dtype=np.float32)) * np.float32(scale)).astype(np.float32).reshape(shape)


def text_config(cfg, vocab):
    d = cfg.text_config()
    d["vocab_size"] = vocab
    d["rope_parameters"]["mrope_section"] = [1, 1, 0]
    d["max_position_embeddings"] = 4096
    return Qwen3_5TextConfig(**{k: v for k, v in d.items() if k != "model_type"})


@torch.no_grad()
def main():
    torch.manual_seed(0)
    out = {}
    # --- RMSNorm (centred) -------------------------------------------------
    for width in (7, 256, 1024):
        x = ramp(np.sin, (17, width))
        w = ramp(np.cos, (width,), 0.1)
        norm = M.Qwen3_5RMSNorm(width, eps=1e-6)
        norm.weight.copy_(torch.from_numpy(w))
        out[f"rms/{width}"] = norm(torch.from_numpy(x)).numpy()
    # --- gated RMSNorm ------------------------------------------------------
    x = ramp(np.sin, (17, 4, 128))
    z = ramp(np.cos, (17, 4, 128), 3.0)
    w = ramp(np.cos, (128,))
    g = M.Qwen3_5RMSNormGated(128, eps=1e-6)
    g.weight.copy_(torch.from_numpy(w))
    out["gated/out"] = g(torch.from_numpy(x), gate=torch.from_numpy(z)).numpy()
    # --- q/k norm + partial RoPE -------------------------------------------
    for tag, hd, rot, heads, kv, seqs, seq in (("hd64", 64, 16, 4, 1, 1, 33),
                                               ("hd256", 256, 64, 4, 1, 2, 10)):
        cfg = plumbing_config()
        tc = text_config(cfg, 64)
        tc.head_dim = hd
        tc.rope_parameters = {"rope_type": "default", "rope_theta": 1e7,
                              "partial_rotary_factor": rot / hd, "mrope_section": [1, 1, 0]}
        rope = M.Qwen3_5TextRotaryEmbedding(tc)
        tokens = seqs * seq
        q = ramp(np.sin, (tokens, heads, hd), 2.0)
        k = ramp(np.cos, (tokens, kv, hd), 2.0)
        qw = ramp(np.cos, (hd,), 0.05)
        kw = ramp(np.sin, (hd,), 0.05)
        qn, kn = M.Qwen3_5RMSNorm(hd), M.Qwen3_5RMSNorm(hd)
        qn.weight.copy_(torch.from_numpy(qw))
        kn.weight.copy_(torch.from_numpy(kw))
        pos = torch.arange(seq).repeat(seqs)[None, :]
        cos, sin = rope(torch.zeros(1, dtype=torch.float32), pos)  # [1, tokens, rot]
        qt = qn(torch.from_numpy(q)).transpose(0, 1)[None]  # [1, heads, tokens, hd]
        kt = kn(torch.from_numpy(k)).transpose(0, 1)[None]
        qe, ke = M.apply_rotary_pos_emb(qt, kt, cos, sin)
        out[f"rope/{tag}/q"] = qe[0].transpose(0, 1).contiguous().numpy()
        out[f"rope/{tag}/k"] = ke[0].transpose(0, 1).contiguous().numpy()
        out[f"rope/{tag}/meta"] = np.array([hd, rot, heads, kv, seqs, seq])
    # --- SwiGLU -------------------------------------------------------------
    gate = ramp(np.sin, (9, 64), 8.0)
    up = ramp(np.cos, (9, 64), 2.0)
    special = np.array([0.0, -0.0, -100.0, 100.0, 1e-30, -1e-30, 80.0, -20.0, 88.0, -88.0,
                        1e-12, 3.0], np.float32)
    gate[0, :special.size] = special
    out["swiglu/gate"] = gate
    out["swiglu/out"] = (ACT2FN["silu"](torch.from_numpy(gate)) * torch.from_numpy(up)).numpy()
    # --- whole 2-layer plumbing backbone ------------------------------------
    cfg = plumbing_config()
    vocab, T, seed = 512, 48, 1234
    W = random_weights(dataclasses.replace(cfg, vocab=vocab), seed=seed)
    model = M.Qwen3_5TextModel(text_config(cfg, vocab)).eval()
    state = {k: torch.from_numpy(v) for k, v in W.items()}
    missing, unexpected = model.load_state_dict(state, strict=False)
    assert not unexpected, unexpected
    assert all("rotary" in m for m in missing), missing
    ids = np.random.default_rng(seed + 1).integers(0, vocab, size=T).astype(np.int64)
    hidden = model(input_ids=torch.from_numpy(ids)[None], use_cache=False).last_hidden_state[0]
    out["model/ids"] = ids.astype(np.int32)
    out["model/hidden"] = hidden.numpy()
    out["model/meta"] = np.array([vocab, T, seed])
    np.savez_compressed(DST, **out)
    print("wrote", DST, sorted(out))


if __name__ == "__main__":
    main()
