"""Seeded synthetic inputs for the BASELINE.json configurations.

Generation rule (all configs): atom counts are drawn first, then tensors, from
one CPU ``torch.Generator().manual_seed(seed)``; tensors are generated in fp32
on the CPU and then cast and moved, so CPU and GPU see identical bits.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass
class SimplicialWorkload:
    name: str
    q: torch.Tensor
    k1: torch.Tensor
    v1: torch.Tensor
    k2: torch.Tensor
    v2: torch.Tensor
    query_valid: torch.Tensor      # (B, N) bool
    pair_key_valid: torch.Tensor   # (B, N) bool
    counts: torch.Tensor           # (B,) int64 valid atoms per molecule

    @property
    def shape(self) -> tuple[int, int, int, int]:
        return tuple(self.q.shape)

    def to(self, device, dtype=None) -> "SimplicialWorkload":
        def mv(t):
            if t.is_floating_point() and dtype is not None:
                t = t.to(dtype)
            return t.to(device)
        return SimplicialWorkload(self.name, *(mv(t) for t in (self.q, self.k1, self.v1, self.k2, self.v2)),
                                  self.query_valid.to(device), self.pair_key_valid.to(device), self.counts)

    def valid_flops(self) -> int:
        """sum_b 4*H*D*n_b^3 (logits 2 n^3 D + value path 2 n^3 D per head)."""
        B, H, N, D = self.shape
        n = self.counts.to(torch.int64)
        return int(4 * H * D * int((n ** 3).sum()))


def qm9_counts(batch: int, gen: torch.Generator) -> torch.Tensor:
    """Config 1: atom counts uniform in [9, 29]."""
    return torch.randint(9, 30, (batch,), generator=gen)


def geom_counts(batch: int, gen: torch.Generator, max_atoms: int = 181) -> torch.Tensor:
    """Config 2: round(44 + 12 z) clipped to [10, 181]."""
    z = torch.randn(batch, generator=gen)
    return torch.clamp(torch.round(44.0 + 12.0 * z), 10, max_atoms).to(torch.int64)


def simplicial_workload(config: str, seed: int | None = None, *, batch: int | None = None,
                        heads: int | None = None) -> SimplicialWorkload:
    """fp32 CPU tensors for config "qm9" (C1) or "geom" (C2); cast/move with ``.to``."""
    if config == "qm9":
        B, H, N, D, seed0, std = 128, 8, 29, 32, 0, 1.0 / math.sqrt(32)
        draw = qm9_counts
    elif config == "geom":
        B, H, N, D, seed0, std = 64, 8, 181, 64, 1, 1.0 / 8.0
        draw = geom_counts
    else:
        raise ValueError(f"unknown simplicial config {config!r}")
    B = batch or B
    H = heads or H
    gen = torch.Generator().manual_seed(seed0 if seed is None else seed)
    counts = draw(B, gen)
    tensors = [torch.randn(B, H, N, D, generator=gen) * std for _ in range(5)]
    valid = torch.arange(N)[None, :] < counts[:, None]
    return SimplicialWorkload(config, *tensors, valid.clone(), valid.clone(), counts)


def random_simplicial(B: int, H: int, N: int, D: int, *, seed: int, counts=None, holes=None,
                      pair_drop: float = 0.0, std: float | None = None):
    """Small random case: returns (q,k1,v1,k2,v2, query_valid, pair_key_valid, pair_valid) fp32 CPU."""
    gen = torch.Generator().manual_seed(seed)
    std = (1.0 / math.sqrt(D)) if std is None else std
    tensors = [torch.randn(B, H, N, D, generator=gen) * std for _ in range(5)]
    key_valid = torch.ones(B, N, dtype=torch.bool)
    if counts is not None:
        for b, n in enumerate(counts):
            key_valid[b, n:] = False
    query_valid = key_valid.clone()
    for b, i in holes or ():
        key_valid[b, i] = False
    pair_valid = None
    if pair_drop > 0:
        pair_valid = torch.rand(B, N, N, generator=gen) >= pair_drop
    return (*tensors, query_valid, key_valid, pair_valid)


@dataclass
class KnnWorkload:
    coords: torch.Tensor            # (B, N, 3) fp32
    pad_mask: torch.Tensor | None   # (B, N) bool, True = padding
    k: int


def knn_workload(seed: int = 2, *, batch: int = 32, atoms: int = 181, k: int = 16) -> KnnWorkload:
    """Config 3: coordinates ~ N(0, 2 A^2) per component, every atom valid."""
    gen = torch.Generator().manual_seed(seed)
    coords = torch.randn(batch, atoms, 3, generator=gen) * math.sqrt(2.0)
    return KnnWorkload(coords, None, k)


@dataclass
class RadiusWorkload:
    frac: torch.Tensor        # (B, N, 3) fp32 fractional coordinates
    lattice: torch.Tensor     # (B, 6) y1 latent [log a, log b, log c, cos alpha, cos beta, cos gamma]
    q: torch.Tensor           # (B, H, N, D) fp32 (cast to the compute dtype)
    k: torch.Tensor
    v: torch.Tensor
    cutoff: float

    def attention_flops(self, n_pairs: int) -> int:
        """4 H D flops per allowed (i, j) pair (q.k and p.v)."""
        B, H, N, D = self.q.shape
        return 4 * H * D * int(n_pairs)


def radius_workload(seed: int = 3, *, cells: int = 8, atoms: int = 512, heads: int = 8, head_dim: int = 64,
                    cutoff: float = 6.0) -> RadiusWorkload:
    """Config 4: frac ~ U[0,1)^3, lengths ~ U[15,30] A, angles ~ U[80,100] deg, q,k,v ~ N(0,1)/8."""
    gen = torch.Generator().manual_seed(seed)
    frac = torch.rand(cells, atoms, 3, generator=gen)
    lengths = 15.0 + 15.0 * torch.rand(cells, 3, generator=gen)
    angles = (80.0 + 20.0 * torch.rand(cells, 3, generator=gen)) * math.pi / 180.0
    lattice = torch.cat([lengths.log(), angles.cos()], dim=-1)
    q, k, v = (torch.randn(cells, heads, atoms, head_dim, generator=gen) / 8.0 for _ in range(3))
    return RadiusWorkload(frac, lattice, q, k, v, cutoff)


@dataclass
class TrunkWorkload:
    x: torch.Tensor        # (B, N, d) fp32 token features
    cond: torch.Tensor     # (B, d) fp32 conditioning embedding
    coords: torch.Tensor   # (B, N, 3) fp32 coordinates, N(0, 2 A^2)
    pad_mask: torch.Tensor  # (B, N) bool, True = padding
    counts: torch.Tensor   # (B,) valid atoms
    d_model: int
    heads: int
    layers: int
    knn_k: int

    def valid_flops(self) -> dict:
        """Algorithmic FLOPs over valid atoms (padded rows are not work):
        simplicial blocks 28 d^2 per token (in_proj 10 d^2, out_proj 2 d^2, MLP 16 d^2) plus 4 H D n^3,
        local blocks 24 d^2 per token plus 4 H D n (k + 1); ada_ln 12 d^2 per molecule and block."""
        d, H = self.d_model, self.heads
        D = d // H
        n = self.counts.to(torch.int64)
        tokens = int(n.sum())
        n_simp = (self.layers + 1) // 2
        n_local = self.layers // 2
        linears = n_simp * 28 * d * d * tokens + n_local * 24 * d * d * tokens
        linears += self.layers * 12 * d * d * int(n.numel())
        simp = n_simp * 4 * H * D * int((n ** 3).sum())
        local = n_local * 4 * H * D * int((n * torch.clamp(n, max=self.knn_k + 1)).sum())
        return {"linears": linears, "simplicial": simp, "local": local, "total": linears + simp + local}


def trunk_workload(seed: int = 4, *, batch: int = 64, atoms: int = 181, d_model: int = 512, heads: int = 8,
                   layers: int = 12, knn_k: int = 32) -> TrunkWorkload:
    """Config 5: GEOM-Drugs atom counts (as config 2), coordinates ~ N(0, 2 A^2) (as config 3), token features
    and conditioning ~ N(0, 1)."""
    gen = torch.Generator().manual_seed(seed)
    counts = geom_counts(batch, gen, atoms)
    pad = torch.arange(atoms)[None, :] >= counts[:, None]
    x = torch.randn(batch, atoms, d_model, generator=gen)
    cond = torch.randn(batch, d_model, generator=gen)
    coords = torch.randn(batch, atoms, 3, generator=gen) * math.sqrt(2.0)
    return TrunkWorkload(x, cond, coords, pad, counts, d_model, heads, layers, knn_k)
