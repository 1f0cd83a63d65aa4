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

The package root exports lazily, so ``matterformer_amd.build`` can be imported
(and the library built) before anything tries to load the library.
"""

_LAZY = {
    "SimplicialAttention": "matterformer_amd.simplicial_attention",
    "SimplicialAttentionMask": "matterformer_amd.simplicial_types",
    "SimplicialFactorizedBias": "matterformer_amd.simplicial_types",
    "SimplicialLowRankAngleResidual": "matterformer_amd.simplicial_types",
    "SimplicialLowRankMessageResidual": "matterformer_amd.simplicial_types",
    "TwoSimplicialAttention": "matterformer_amd.simplicial_attention",
}

__all__ = sorted(_LAZY)


def __getattr__(name):
    module = _LAZY.get(name)
    if module is None:
        raise AttributeError(f"module 'matterformer_amd' has no attribute {name!r}")
    import importlib

    return getattr(importlib.import_module(module), name)
