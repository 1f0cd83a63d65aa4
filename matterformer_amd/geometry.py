"""Geometry adapters whose pair features come from one HIP pass (mf_geometry_features).

Mirror of ``matterformer.geometry.adapters`` (src/matterformer/geometry/adapters.py): the same class names,
constructor and forward signatures and the same ``GeometryFeatures`` (:12-21).

  NonPeriodicGeometryAdapter.forward   :83-125
  PeriodicGeometryAdapter.forward      :151-212 (27 / 125 images, argmin under the lattice metric)

On GPU tensors the pair tensors (delta, d2, d, d_norm) are written by one kernel that evaluates the images
in registers: the reference's [B, N, N, 27, 3] image tensor (:176-189) is never formed.  ``forward`` can
also return the cutoff neighbour mask of the same pass (``radius_cutoff=``, in ``extras["radius_mask_bits"]``,
mf_radius_mask's layout), which local attention and the kNN / radius consumers read.  The per-molecule
normalisers (rms radius, cell scale) and the lattice conversions are small torch reductions.  CPU tensors take
the reference's own torch formulation (as the reference does for them).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from itertools import product

import torch
from torch import nn

from matterformer_amd.geometry_ops import lattice_terms


@dataclass
class GeometryFeatures:
    pair_delta: torch.Tensor
    pair_dist: torch.Tensor
    pair_dist2: torch.Tensor
    pair_dist_norm: torch.Tensor
    pair_mask: torch.Tensor
    global_geom: torch.Tensor
    kind: str
    extras: dict[str, torch.Tensor] = field(default_factory=dict)


def lattice_latent_to_y1(lattice: torch.Tensor, lattice_repr: str = "y1") -> torch.Tensor:
    """lattice.py:65-91,103-131: the clamped y1 latent (y1) or y1 recovered from the Gram matrix (ltri)."""
    return lattice_terms(lattice, lattice_repr)[1]


_METRICS: dict = {}


def _identity_metric(batch: int, device: torch.device) -> torch.Tensor:
    """torch.eye(3) expanded over the batch (the non-periodic adapter's metric), one 3x3 tensor per device."""
    key = (device.type, device.index)
    eye = _METRICS.get(key)
    if eye is None:
        eye = torch.eye(3, device=device, dtype=torch.float32)
        _METRICS[key] = eye
    return eye.expand(batch, -1, -1)


class BaseGeometryAdapter(nn.Module):
    geometry_kind: str = "base"

    @staticmethod
    def _valid_atom_mask(coords: torch.Tensor, pad_mask: torch.Tensor | None) -> torch.Tensor:
        B, N = coords.shape[:2]
        if pad_mask is None:
            return torch.ones(B, N, device=coords.device, dtype=torch.bool)
        if pad_mask.shape != (B, N):
            raise ValueError(f"pad_mask must have shape {(B, N)}, got {tuple(pad_mask.shape)}")
        return ~pad_mask.bool()

    @staticmethod
    def _pair_mask_from_valid(valid: torch.Tensor) -> torch.Tensor:
        return valid[:, :, None] & valid[:, None, :]

    @staticmethod
    def _masked(t: torch.Tensor, pair_mask: torch.Tensor) -> torch.Tensor:
        m = pair_mask
        while m.ndim < t.ndim:
            m = m.unsqueeze(-1)
        return torch.where(m, t, torch.zeros_like(t))

    @staticmethod
    def _hip_features(coords, pad_mask, scale, gram, pbc_radius, radius_cutoff):
        """One mf_geometry_features call: the pair tensors, the valid-pair mask and (scale None: the
        non-periodic rms radius, computed in the same call) the normaliser."""
        from matterformer_amd import _native

        B, N, _ = coords.shape
        dev = coords.device
        c = coords.float().contiguous()
        # a bool mask is read as its bytes (0 / 1)
        pad = None if pad_mask is None else pad_mask.to(torch.bool).contiguous()
        delta = torch.empty(B, N, N, 3, device=dev, dtype=torch.float32)
        d2 = torch.empty(B, N, N, device=dev, dtype=torch.float32)
        dist = torch.empty_like(d2)
        dnorm = torch.empty_like(d2)
        pair_mask = torch.empty(B, N, N, device=dev, dtype=torch.uint8)
        bits = None
        if radius_cutoff is not None:
            bits = torch.empty(B, N, (N + 31) // 32, device=dev, dtype=torch.int32)
        g = None if gram is None else gram.float().contiguous()
        rms_mode = scale is None
        sc = torch.empty(B, device=dev, dtype=torch.float32) if rms_mode else scale.float().contiguous()
        args = _native.MfGeometryArgs(
            coords=c.data_ptr(), gram=_native.ptr(g), scale=sc.data_ptr(), pad_mask=_native.ptr(pad),
            pair_delta=delta.data_ptr(), pair_dist2=d2.data_ptr(), pair_dist=dist.data_ptr(),
            pair_dist_norm=dnorm.data_ptr(), mask_bits=_native.ptr(bits),
            cutoff=float(radius_cutoff) if radius_cutoff is not None else 0.0, batch=B, atoms=N,
            pbc_radius=int(pbc_radius), pair_mask=pair_mask.data_ptr(),
            scale_mode=_native.MF_SCALE_RMS if rms_mode else _native.MF_SCALE_GIVEN)
        with torch.cuda.device(dev):
            _native.check(_native.lib().mf_geometry_features(args, _native.current_stream(dev)),
                          "mf_geometry_features")
        return delta, dist, d2, dnorm, bits, pair_mask.view(torch.bool), sc


class NonPeriodicGeometryAdapter(BaseGeometryAdapter):
    geometry_kind = "nonperiodic"

    def forward(self, coords: torch.Tensor, pad_mask: torch.Tensor | None = None,
                lattice: torch.Tensor | None = None, *, radius_cutoff: float | None = None) -> GeometryFeatures:
        if coords.ndim != 3 or coords.shape[-1] != 3:
            raise ValueError(f"coords must have shape (B, N, 3), got {tuple(coords.shape)}")
        if lattice is not None:
            raise ValueError("lattice must be None for NonPeriodicGeometryAdapter")
        coords = coords.float()
        extras = {"metric": _identity_metric(coords.shape[0], coords.device)}
        if coords.device.type == "cuda":
            if pad_mask is not None and pad_mask.shape != coords.shape[:2]:
                raise ValueError(f"pad_mask must have shape {tuple(coords.shape[:2])}, got {tuple(pad_mask.shape)}")
            # one call: rms radius, pair tensors and the valid-pair mask
            delta, dist, d2, dnorm, bits, pair_mask, rms = self._hip_features(coords, pad_mask, None, None, 0,
                                                                              radius_cutoff)
            if bits is not None:
                extras["radius_mask_bits"] = bits
        else:
            valid = self._valid_atom_mask(coords, pad_mask)
            pair_mask = self._pair_mask_from_valid(valid)
            sq_norm = coords.square().sum(dim=-1)
            denom = valid.sum(dim=1).clamp_min(1)
            rms = torch.sqrt(((sq_norm * valid.to(sq_norm.dtype)).sum(dim=1) / denom).clamp_min(1e-8))
            delta = coords[:, :, None, :] - coords[:, None, :, :]
            d2 = delta.square().sum(dim=-1).clamp_min(0.0)
            dist = torch.sqrt(d2)
            dnorm = dist / rms[:, None, None].clamp_min(1e-8)
            delta, dist, d2, dnorm = (self._masked(t, pair_mask) for t in (delta, dist, d2, dnorm))
            if radius_cutoff is not None:
                extras["radius_mask"] = pair_mask & (d2 <= float(radius_cutoff) ** 2)
        return GeometryFeatures(pair_delta=delta, pair_dist=dist, pair_dist2=d2, pair_dist_norm=dnorm,
                                pair_mask=pair_mask, global_geom=rms[:, None], kind=self.geometry_kind, extras=extras)


class PeriodicGeometryAdapter(BaseGeometryAdapter):
    geometry_kind = "periodic"

    def __init__(self, pbc_radius: int = 1, lattice_repr: str = "y1") -> None:
        super().__init__()
        if pbc_radius not in {1, 2}:
            raise ValueError(f"pbc_radius must be 1 or 2, got {pbc_radius}")
        self.pbc_radius = int(pbc_radius)
        self.lattice_repr = lattice_repr.lower()
        offsets = torch.tensor(list(product(range(-self.pbc_radius, self.pbc_radius + 1), repeat=3)),
                               dtype=torch.float32)
        self.register_buffer("_pbc_offsets", offsets.view(1, 1, 1, offsets.shape[0], 3), persistent=False)

    def forward(self, coords: torch.Tensor, pad_mask: torch.Tensor | None = None,
                lattice: torch.Tensor | None = None, *, radius_cutoff: float | None = None) -> GeometryFeatures:
        if coords.ndim != 3 or coords.shape[-1] != 3:
            raise ValueError(f"coords must have shape (B, N, 3), got {tuple(coords.shape)}")
        if lattice is None:
            raise ValueError("lattice is required for PeriodicGeometryAdapter")
        if lattice.ndim != 2 or lattice.shape[-1] != 6:
            raise ValueError(f"lattice must have shape (B, 6), got {tuple(lattice.shape)}")
        if lattice.shape[0] != coords.shape[0]:
            raise ValueError(f"lattice batch {lattice.shape[0]} does not match coords batch {coords.shape[0]}")
        coords = coords.float()
        lattice = lattice.float()
        # adapters.py:173-174,192 (one mf_lattice_terms launch on the GPU)
        gram, y1, cell_scale = lattice_terms(lattice, self.lattice_repr)
        extras = {"metric": gram, "cell_scale": cell_scale[:, None]}
        if coords.device.type == "cuda":
            if pad_mask is not None and pad_mask.shape != coords.shape[:2]:
                raise ValueError(f"pad_mask must have shape {tuple(coords.shape[:2])}, got {tuple(pad_mask.shape)}")
            delta, dist, d2, dnorm, bits, pair_mask, _ = self._hip_features(coords, pad_mask, cell_scale, gram,
                                                                            self.pbc_radius, radius_cutoff)
            if bits is not None:
                extras["radius_mask_bits"] = bits
        else:
            valid = self._valid_atom_mask(coords, pad_mask)
            pair_mask = self._pair_mask_from_valid(valid)
            delta0 = coords[:, :, None, :] - coords[:, None, :, :]
            images = delta0[:, :, :, None, :] + self._pbc_offsets.to(coords.device, coords.dtype)
            d2_images = torch.einsum("bnmki,bij,bnmkj->bnmk", images, gram, images)
            idx = d2_images.argmin(dim=-1, keepdim=True)
            d2 = torch.gather(d2_images, -1, idx).squeeze(-1).clamp_min(0.0)
            delta = torch.gather(images, 3, idx[..., None].expand(-1, -1, -1, 1, 3)).squeeze(3)
            dist = torch.sqrt(d2)
            dnorm = dist / cell_scale[:, None, None]
            delta, dist, d2, dnorm = (self._masked(t, pair_mask) for t in (delta, dist, d2, dnorm))
            if radius_cutoff is not None:
                extras["radius_mask"] = pair_mask & (d2 <= float(radius_cutoff) ** 2)
        return GeometryFeatures(pair_delta=delta, pair_dist=dist, pair_dist2=d2, pair_dist_norm=dnorm,
                                pair_mask=pair_mask, global_geom=y1, kind=self.geometry_kind, extras=extras)
