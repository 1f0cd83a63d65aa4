"""Compatibility re-exports (mirror of src/matterformer/models/attention_triton.py:1-19).

The names keep the reference's "triton" spelling; they resolve to the HIP backend.
"""

from __future__ import annotations

from matterformer_amd.hip_simplicial_attention import (
    SUPPORTED_SIMPLICIAL_PRECISIONS,
    TRITON_AVAILABLE,
    normalize_simplicial_precision,
    triton_block_d_for_head_dim,
    triton_simplicial_attention_backward,
    triton_simplicial_attention_forward,
)

__all__ = [
    "TRITON_AVAILABLE",
    "SUPPORTED_SIMPLICIAL_PRECISIONS",
    "normalize_simplicial_precision",
    "triton_block_d_for_head_dim",
    "triton_simplicial_attention_backward",
    "triton_simplicial_attention_forward",
]
