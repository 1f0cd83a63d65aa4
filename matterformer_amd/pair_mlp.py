"""The factorized geometry-bias MLPs on the GPU: SimplicialGeometryBias._compute_factorized_terms
(src/matterformer/models/transformer.py:702-717) as one mf_pair_mlp_bias pass over the valid pairs.

Used for inference calls (the kernel has no backward): GPU features, fp32 weights and features, materialised
LazyLinear layers (their first call runs the torch formulation, which draws their weights in the reference's
order), non-periodic spoke features (no Fourier / global terms), rbf <= 29, hidden a multiple of 16 <= 256,
heads <= 16.  Everything else takes the torch formulation.
"""

from __future__ import annotations

import torch
from torch.nn.parameter import UninitializedParameter

from matterformer_amd import _native


def _mlp_parts(mlp):
    first, act, last = mlp[0], mlp[1], mlp[2]
    return first, act, last


def serves(module, geom_features) -> bool:
    g = geom_features
    if g.pair_delta.device.type != "cuda":
        return False
    mlps = (module.spoke_bias_u_mlp, module.spoke_bias_v_mlp, module.pair_bias_w_mlp)
    params = [prm for m in mlps for prm in m.parameters()]
    if any(isinstance(prm, UninitializedParameter) for prm in params):
        return False
    if torch.is_grad_enabled() and (any(prm.requires_grad for prm in params) or g.pair_delta.requires_grad
                                    or g.pair_dist_norm.requires_grad):
        return False
    if module.use_periodic_features and g.kind == "periodic":
        return False
    if not isinstance(mlps[0][1], torch.nn.SiLU):
        return False
    R = module.edge_bias_n_rbf
    hidden = mlps[0][0].out_features
    if not (1 <= R <= 29 and hidden % 16 == 0 and 16 <= hidden <= 256 and 1 <= module.n_heads <= 16):
        return False
    if any(m[0].out_features != hidden or m[0].bias is None or m[2].bias is None for m in mlps):
        return False
    if mlps[0][0].in_features != 3 + R or mlps[1][0].in_features != 3 + R or mlps[2][0].in_features != R:
        return False
    tensors = [g.pair_delta, g.pair_dist_norm] + params
    return all(t.dtype == torch.float32 for t in tensors)


def factorized_terms(module, geom_features):
    """(u, v, w) [B, H, N, N] fp32, diagonal and invalid pairs zero."""
    g = geom_features
    B, N = g.pair_delta.shape[:2]
    H = module.n_heads
    dev = g.pair_delta.device
    delta = g.pair_delta.contiguous()
    dnorm = g.pair_dist_norm.contiguous()
    mask = g.pair_mask.to(torch.uint8).contiguous()
    centers = module._edge_rbf_centers.to(device=dev, dtype=torch.float32).contiguous()
    gamma = module._edge_rbf_gamma_value
    outs = [torch.empty(B, H, N, N, device=dev, dtype=torch.float32) for _ in range(3)]
    keep = [delta, dnorm, mask, centers]
    fields = {}
    for name, mlp in zip("uvw", (module.spoke_bias_u_mlp, module.spoke_bias_v_mlp, module.pair_bias_w_mlp)):
        first, _, last = _mlp_parts(mlp)
        ts = [first.weight.contiguous(), first.bias.contiguous(), last.weight.contiguous(), last.bias.contiguous()]
        keep += ts
        for t, key in zip(ts, ("w1", "b1", "w2", "b2")):
            fields[f"{name}_{key}"] = t.data_ptr()
    args = _native.MfPairMlpArgs(
        pair_delta=delta.data_ptr(), pair_dist_norm=dnorm.data_ptr(), pair_mask=mask.data_ptr(),
        rbf_centers=centers.data_ptr(), rbf_gamma=gamma, u_out=outs[0].data_ptr(), v_out=outs[1].data_ptr(),
        w_out=outs[2].data_ptr(), batch=B, atoms=N, rbf=int(centers.numel()), hidden=module.spoke_bias_u_mlp[0].out_features,
        heads=H, **fields)
    with torch.cuda.device(dev):
        _native.check(_native.lib().mf_pair_mlp_bias(args, _native.current_stream(dev)), "mf_pair_mlp_bias")
    return tuple(outs)
