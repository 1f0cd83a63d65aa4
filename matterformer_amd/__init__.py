"""MI355X-native (gfx950) kernels for Matterformer's geometric-attention hot path.

Public modules:
  matterformer_amd.simplicial_attention      SimplicialAttention & friends (mirror of
                                             matterformer.models.simplicial_attention)
  matterformer_amd.hip_simplicial_attention  launcher (mirror of
                                             matterformer.models.triton_simplicial_attention)
  matterformer_amd.attention / attention_triton / triton_regular_attention
                                             re-export shims of the reference
  matterformer_amd.geometry_ops              kNN top-k, radius mask, radius attention
The kernels live in libmf_hip.so (C ABI: include/mf_capi.h), built by
``python -m matterformer_amd.build``.
"""

from matterformer_amd.simplicial_attention import (  # noqa: F401
    SimplicialAttention,
    SimplicialAttentionMask,
    SimplicialFactorizedBias,
    SimplicialLowRankAngleResidual,
    SimplicialLowRankMessageResidual,
    TwoSimplicialAttention,
)
