"""Backbone weights as a name -> array dict, keyed like the checkpoint with the
``language_model.`` prefix removed and stored as in the file (PyTorch
``[out, in]``, i.e. the reference's Julia ``(in, out)`` in the same memory).

``read_checkpoint`` follows ``read_native_weights`` (``src/safetensors.jl:3-35``)
and the name canonicalisation of ``QwenBackbone`` (``src/backbone.jl:107-134``);
``read_checkpoint_tensors`` is the device loader that keeps BF16 weights in bf16;
``random_weights`` builds the synthetic random-init backbones.
"""
from __future__ import annotations

import json
import os

import numpy as np

from .config import BackboneConfig


def layer_shapes(cfg: BackboneConfig, index: int) -> dict:
    """Tensor shapes of one layer, checkpoint layout."""
    p = f"layers.{index}."
    H, I = cfg.hidden, cfg.intermediate
    shapes = {
        p + "input_layernorm.weight": (H,),
        p + "post_attention_layernorm.weight": (H,),
        p + "mlp.gate_proj.weight": (I, H),
        p + "mlp.up_proj.weight": (I, H),
        p + "mlp.down_proj.weight": (H, I),
    }
    kind = cfg.layer_types[index]
    if kind == "full_attention":
        hd = cfg.head_dim
        shapes.update({
            p + "self_attn.q_proj.weight": (2 * hd * cfg.heads, H),
            p + "self_attn.k_proj.weight": (hd * cfg.kv_heads, H),
            p + "self_attn.v_proj.weight": (hd * cfg.kv_heads, H),
            p + "self_attn.o_proj.weight": (H, hd * cfg.heads),
            p + "self_attn.q_norm.weight": (hd,),
            p + "self_attn.k_norm.weight": (hd,),
        })
    elif kind == "linear_attention":
        kw = cfg.key_dim * cfg.key_heads
        vw = cfg.value_dim * cfg.value_heads
        shapes.update({
            p + "linear_attn.in_proj_qkv.weight": (2 * kw + vw, H),
            p + "linear_attn.in_proj_z.weight": (vw, H),
            p + "linear_attn.in_proj_a.weight": (cfg.value_heads, H),
            p + "linear_attn.in_proj_b.weight": (cfg.value_heads, H),
            p + "linear_attn.conv1d.weight": (2 * kw + vw, 1, cfg.conv_kernel),
            p + "linear_attn.A_log": (cfg.value_heads,),
            p + "linear_attn.dt_bias": (cfg.value_heads,),
            p + "linear_attn.norm.weight": (cfg.value_dim,),
            p + "linear_attn.out_proj.weight": (H, vw),
        })
    else:
        raise ValueError(f"Unsupported layer type {kind}.")
    return shapes


def all_shapes(cfg: BackboneConfig) -> dict:
    shapes = {"embed_tokens.weight": (cfg.vocab, cfg.hidden)}
    for i in range(len(cfg.layer_types)):
        shapes.update(layer_shapes(cfg, i))
    shapes["norm.weight"] = (cfg.hidden,)
    return shapes


def random_weights(cfg: BackboneConfig, seed: int = 0, std: float = 0.02) -> dict:
    """Every tensor ~ N(0, std) in fp32 from ``numpy.random.default_rng(seed)``,
    drawn in the order of :func:`all_shapes` (deterministic across machines)."""
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in all_shapes(cfg).items():
        out[name] = (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)
    return out


def random_device_weights(cfg: BackboneConfig, seed: int = 0, device="cuda:0", dtype=None,
                          std: float = 0.02) -> dict:
    """Every tensor ~ N(0, std), generated on the device with a seeded torch
    generator (fast at full model size; values differ from :func:`random_weights`)."""
    import torch
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    out = {}
    for name, shape in all_shapes(cfg).items():
        t = torch.randn(shape, generator=gen, device=device, dtype=torch.float32) * std
        out[name] = t.to(dtype) if dtype is not None else t
    return out


def _checkpoint_files(directory: str) -> list:
    """The safetensors files of a local checkpoint: ``model.safetensors`` or the
    shards named by ``model.safetensors.index.json`` (``src/safetensors.jl:3-17``)."""
    single = os.path.join(directory, "model.safetensors")
    if os.path.isfile(single):
        return ["model.safetensors"]
    with open(os.path.join(directory, "model.safetensors.index.json")) as f:
        files = sorted(set(json.load(f)["weight_map"].values()))
    for fname in files:
        if os.path.isabs(fname) or ".." in fname.split("/"):
            raise ValueError(f"Unsafe shard path {fname}.")
    return files


def _strip(name: str):
    at = name.find("language_model.")
    return None if at < 0 else name[at + len("language_model."):]


def read_checkpoint_tensors(directory: str, device="cpu") -> dict:
    """Every ``language_model.*`` tensor of a local safetensors checkpoint as a
    torch tensor in its stored dtype, loaded straight onto ``device``: BF16
    weights stay bf16 (no fp32 widening, half the bytes of the widened load of
    ``src/safetensors.jl:28-30``).  Safe loader: nothing in the file is executed."""
    from safetensors.torch import load_file

    out = {}
    for fname in _checkpoint_files(directory):
        for name, value in load_file(os.path.join(directory, fname), device=str(device)).items():
            key = _strip(name)
            if key is not None:
                out[key] = value
    return out


def read_checkpoint(directory: str) -> dict:
    """Load every ``language_model.*`` tensor of a local safetensors checkpoint
    (single file or sharded index) widened to fp32 numpy (``src/safetensors.jl:28-30``)."""
    import torch

    out = {}
    for key, value in read_checkpoint_tensors(directory, device="cpu").items():
        if value.dtype == torch.bfloat16:  # widen: bits << 16, exact
            bits = value.contiguous().view(torch.int16).numpy().view(np.uint16)
            out[key] = (bits.astype(np.uint32) << 16).view(np.float32)
        else:
            out[key] = value.to(torch.float32).numpy()
    return out
