"""Shared by the trunk tests: the configs[4] trunk built as tests/golden/make_golden.py built the reference's.

Seeded construction (torch.manual_seed(seed)) draws the reference's initial weights because the blocks
create the same modules in the same order; ada_ln's last layer is then overwritten with
N(0, ada_std^2) draws from torch.Generator().manual_seed(seed + 100), block by block, weight then bias,
exactly as the fixture script does for the reference blocks.
"""

from pathlib import Path

import numpy as np
import torch

from matterformer_amd.trunk import AlternatingTrunk

GOLDEN = Path(__file__).resolve().parent / "golden" / "trunk_alternating_b4.npz"


def load():
    return np.load(GOLDEN)


def build_trunk(z, **kw):
    B, d, H, L, k = (int(v) for v in z["shape"])
    seed = int(z["seed"])
    torch.manual_seed(seed)
    trunk = AlternatingTrunk(d, H, L, knn_k=k, **kw)
    ada = torch.Generator().manual_seed(seed + 100)
    std = float(z["ada_std"])
    for blk in trunk.blocks:
        lin = blk.ada_ln[-1]
        lin.weight.data.copy_(torch.randn(lin.weight.shape, generator=ada) * std)
        lin.bias.data.copy_(torch.randn(lin.bias.shape, generator=ada) * std)
    return trunk


def inputs(z):
    return (torch.from_numpy(z["x"]), torch.from_numpy(z["cond"]), torch.from_numpy(z["coords"]),
            torch.from_numpy(z["pad_mask"]))


def valid_rel_err(out, z):
    pad = z["pad_mask"]
    got = np.asarray(out, dtype=np.float64)[~pad]
    ref = z["out"].astype(np.float64)[~pad]
    return float(np.linalg.norm(got - ref) / np.linalg.norm(ref))


def geometry_trunk(mode="angle_low_rank", message_mode="low_rank", *, d=64, H=4, L=4, k=8, seed=11, **kw):
    """A small alternating trunk with a NonPeriodicGeometryAdapter and a SimplicialGeometryBias whose output
    layers (zero at construction) and ada_ln layers are drawn from N(0, 0.3^2) / N(0, 0.05^2), so every bias,
    residual and gate term reaches the output; the LazyLinear layers are materialised by one CPU forward."""
    from matterformer_amd.geometry import NonPeriodicGeometryAdapter
    from matterformer_amd.geometry_bias import SimplicialGeometryBias

    torch.manual_seed(seed)
    bias = SimplicialGeometryBias(H, mode=mode, edge_bias_hidden_dim=32, edge_bias_n_rbf=12,
                                  angle_residual_rank=8, message_mode=message_mode, message_rank=8)
    trunk = AlternatingTrunk(d, H, L, knn_k=k, simplicial_message_mode=message_mode, simplicial_message_rank=8,
                             geometry_adapter=NonPeriodicGeometryAdapter(), simplicial_geometry_bias=bias, **kw)
    x, cond, coords, pad, sigma = geometry_inputs(d, seed)
    with torch.no_grad():
        trunk(x[:1], cond[:1], coords[:1], pad[:1], sigma=sigma[:1])
    gen = torch.Generator().manual_seed(seed + 1)
    for name, prm in bias.named_parameters():
        if name.endswith(".2.weight") or name.endswith(".2.bias"):
            prm.data.copy_(torch.randn(prm.shape, generator=gen) * 0.3)
    for blk in trunk.blocks:
        lin = blk.ada_ln[-1]
        lin.weight.data.copy_(torch.randn(lin.weight.shape, generator=gen) * 0.05)
        lin.bias.data.copy_(torch.randn(lin.bias.shape, generator=gen) * 0.05)
    return trunk


def geometry_inputs(d=64, seed=11, B=3, N=29):
    gen = torch.Generator().manual_seed(seed + 2)
    counts = torch.tensor([N, N - 9, 13])[:B]
    pad = torch.arange(N)[None, :] >= counts[:, None]
    x = torch.randn(B, N, d, generator=gen)
    cond = torch.randn(B, d, generator=gen)
    coords = torch.randn(B, N, 3, generator=gen) * 1.4
    sigma = torch.rand(B, generator=gen) * 2.0 + 0.05
    return x, cond, coords, pad, sigma
