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
