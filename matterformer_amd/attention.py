"""Compatibility re-exports (mirror of src/matterformer/models/attention.py:1-37)."""

from __future__ import annotations

from matterformer_amd.hip_simplicial_attention import (
    SUPPORTED_SIMPLICIAL_PRECISIONS,
    TRITON_AVAILABLE,
    normalize_simplicial_precision,
    triton_block_d_for_head_dim,
    triton_simplicial_attention_backward,
    triton_simplicial_attention_forward,
)
from matterformer_amd.simplicial_attention import (
    SimplicialAttention,
    SimplicialAttentionMask,
    SimplicialFactorizedBias,
    SimplicialLowRankAngleResidual,
    SimplicialLowRankMessageResidual,
    TwoSimplicialAttention,
    _TritonTwoSimplicialAttentionFunction,
    simplicial_attention_torch_from_projected,
)

__all__ = [
    "TRITON_AVAILABLE",
    "SUPPORTED_SIMPLICIAL_PRECISIONS",
    "SimplicialAttention",
    "SimplicialAttentionMask",
    "SimplicialFactorizedBias",
    "SimplicialLowRankAngleResidual",
    "SimplicialLowRankMessageResidual",
    "TwoSimplicialAttention",
    "_TritonTwoSimplicialAttentionFunction",
    "normalize_simplicial_precision",
    "simplicial_attention_torch_from_projected",
    "triton_block_d_for_head_dim",
    "triton_simplicial_attention_backward",
    "triton_simplicial_attention_forward",
]
