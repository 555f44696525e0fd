"""Backbone configuration: parsing of a checkpoint ``config.json`` and the
synthetic Qwen3.5-style shapes used by the tests and the benchmark.

Mirrors the config handling of ``QwenBackbone`` (``src/backbone.jl:74-106``):
the same fields, the same validation and the same ArgumentError conditions
(raised here as ``ValueError``).
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass, field, asdict

import numpy as np

QWEN_BACKBONE_TYPES = ("qwen3_5", "qwen3_5_text", "qwen3_8", "qwen3_8_text")  # src/backbone.jl:72


@dataclass(frozen=True)
class BackboneConfig:
    hidden: int
    head_dim: int
    heads: int
    kv_heads: int
    key_heads: int
    value_heads: int
    key_dim: int
    value_dim: int
    eps: float
    rope_theta: float
    rotary_dim: int
    layer_types: tuple = field(default_factory=tuple)
    intermediate: int = 0
    vocab: int = 0
    conv_kernel: int = 4

    def __post_init__(self):
        if self.value_heads % self.key_heads:
            raise ValueError("Value heads must be a multiple of key heads.")
        if self.heads % self.kv_heads:
            raise ValueError("Query heads must be a multiple of KV heads.")
        if self.rotary_dim % 2 or self.rotary_dim > self.head_dim:
            raise ValueError("rotary_dim must be even and at most head_dim.")

    def as_dict(self) -> dict:
        d = asdict(self)
        d["layer_types"] = list(self.layer_types)
        return d

    def text_config(self) -> dict:
        """The Hugging Face ``text_config`` this configuration corresponds to."""
        return {
            "model_type": "qwen3_5_text",
            "vocab_size": self.vocab,
            "hidden_size": self.hidden,
            "intermediate_size": self.intermediate,
            "num_hidden_layers": len(self.layer_types),
            "num_attention_heads": self.heads,
            "num_key_value_heads": self.kv_heads,
            "head_dim": self.head_dim,
            "hidden_act": "silu",
            "rms_norm_eps": self.eps,
            "attention_bias": False,
            "rope_parameters": {"rope_type": "default", "rope_theta": self.rope_theta,
                                "partial_rotary_factor": self.rotary_dim / self.head_dim},
            "linear_conv_kernel_dim": self.conv_kernel,
            "linear_key_head_dim": self.key_dim,
            "linear_value_head_dim": self.value_dim,
            "linear_num_key_heads": self.key_heads,
            "linear_num_value_heads": self.value_heads,
            "layer_types": list(self.layer_types),
        }


def config_from_text_config(cfg: dict, vocab: int | None = None) -> BackboneConfig:
    """``src/backbone.jl:84-106``."""
    if cfg.get("attention_bias", False):
        raise ValueError("Attention biases are not supported.")
    if cfg.get("hidden_act", "silu") != "silu":
        raise ValueError("Expected SiLU activation.")
    rope = cfg["rope_parameters"]
    if rope.get("rope_type", "default") != "default":
        raise ValueError("Only default RoPE is supported.")
    return BackboneConfig(
        hidden=int(cfg["hidden_size"]),
        head_dim=int(cfg["head_dim"]),
        heads=int(cfg["num_attention_heads"]),
        kv_heads=int(cfg["num_key_value_heads"]),
        key_heads=int(cfg["linear_num_key_heads"]),
        value_heads=int(cfg["linear_num_value_heads"]),
        key_dim=int(cfg["linear_key_head_dim"]),
        value_dim=int(cfg["linear_value_head_dim"]),
        eps=float(np.float32(cfg["rms_norm_eps"])),
        rope_theta=float(np.float32(rope["rope_theta"])),
        # only rope_parameters.partial_rotary_factor is read (src/backbone.jl:101)
        rotary_dim=int(cfg["head_dim"] * rope.get("partial_rotary_factor", 1.0)),
        layer_types=tuple(cfg["layer_types"]),
        intermediate=int(cfg.get("intermediate_size", 0)),
        vocab=int(cfg.get("vocab_size", 0) if vocab is None else vocab),
        conv_kernel=int(cfg.get("linear_conv_kernel_dim", 4)),
    )


def load_config(directory: str) -> BackboneConfig:
    """Read ``config.json`` of a local checkpoint directory (``src/backbone.jl:78-84``)."""
    with open(os.path.join(directory, "config.json")) as f:
        source = json.load(f)
    if source.get("model_type") not in QWEN_BACKBONE_TYPES:
        raise ValueError("QwenBackbone supports Qwen3.5 / Qwen3.8 text backbones, "
                         f"got {source.get('model_type')}.")
    return config_from_text_config(source.get("text_config", source))


def hybrid_layer_types(depth: int, interval: int = 4) -> tuple:
    """3:1 DeltaNet:full pattern, full attention at ``(i+1) % interval == 0``."""
    return tuple("full_attention" if (i + 1) % interval == 0 else "linear_attention"
                 for i in range(depth))


def plumbing_config() -> BackboneConfig:
    """2-layer CPU-runnable backbone: hidden 256, 4 Q / 1 KV heads of 64, rotary 16,
    theta 1e7, intermediate 768, vocab 4096, DeltaNet keys 2x128 / values 4x128."""
    return BackboneConfig(hidden=256, head_dim=64, heads=4, kv_heads=1, key_heads=2,
                          value_heads=4, key_dim=128, value_dim=128,
                          eps=float(np.float32(1e-6)), rope_theta=1e7, rotary_dim=16,
                          layer_types=("linear_attention", "full_attention"),
                          intermediate=768, vocab=4096)


def synthetic_inference_config() -> BackboneConfig:
    """The shapes of the reference's inference benchmark model
    (``benchmark/synthetic.jl:3-28``): 4 layers, DeltaNet x3 then full attention
    (full at ``i % 4 == 0``, 1-based), hidden 256, intermediate 512, 4 Q / 2 KV
    heads of 64 (rotary 16, theta 1e4), DeltaNet keys 2x128 / values 4x128,
    vocab 256."""
    return BackboneConfig(hidden=256, head_dim=64, heads=4, kv_heads=2, key_heads=2,
                          value_heads=4, key_dim=128, value_dim=128,
                          eps=float(np.float32(1e-6)), rope_theta=1e4, rotary_dim=16,
                          layer_types=hybrid_layer_types(4), intermediate=512, vocab=256)


def qwen35_08b_config(depth: int = 24) -> BackboneConfig:
    """Qwen3.5-0.8B-like shapes: hidden 1024, 8 Q / 2 KV heads of 256 (rotary 64),
    DeltaNet 16 key heads x 128 and 16 value heads x 128, intermediate 3584,
    vocab 248320, 3:1 DeltaNet:full."""
    return BackboneConfig(hidden=1024, head_dim=256, heads=8, kv_heads=2, key_heads=16,
                          value_heads=16, key_dim=128, value_dim=128,
                          eps=float(np.float32(1e-6)), rope_theta=1e7, rotary_dim=64,
                          layer_types=hybrid_layer_types(depth), intermediate=3584,
                          vocab=248320)
