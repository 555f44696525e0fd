"""qdc_amd -- MI355X-native fused row kernels of the QwenDecisionCore.jl backbone.

``ops`` holds the device operators (embedding gather, zero-centred RMSNorm,
residual + RMSNorm, q/k norm + partial RoPE, gated RMSNorm, SwiGLU), each one
launch of the HIP library ``lib/libqdc_hip.so``; ``backbone`` runs
``backbone_hidden`` with them; ``graphs`` serves repeated single-sequence
last-token calls from recorded HIP graphs; ``config`` and ``weights`` describe
and build backbones.
"""
from ._lib import LIB_PATH, QDCError, version  # noqa: F401

__all__ = ["LIB_PATH", "QDCError", "version"]
