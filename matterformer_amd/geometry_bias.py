"""Simplicial geometry bias: the factorized / low-rank logit and message terms of simplicial attention built
from the geometry adapters' pair features, and the attention-mask builder of the reference trunk.

Mirror of ``matterformer.models.transformer`` (src/matterformer/models/transformer.py):

  _softplus_inverse                          :31-33
  build_simplicial_attention_mask            :36-73  (``_build_simplicial_attention_mask``)
  _GeometryBiasBase                          :319-396 (noise gate, pair masking, diagonal, expansion)
  SimplicialGeometryBias                     :516-996

The same class, parameter and buffer names, constructor and method signatures, and the same submodule
creation and first-call order, so a seeded construction plus the first forward draws the reference's weights
(the LazyLinear layers materialise on their first call) and a reference state dict loads.

On GPU tensors, ``_compute_factorized_terms`` runs the three pairwise MLPs (spoke u, spoke v, pair w:
LazyLinear -> SiLU -> Linear over the [B, N, N, F] features) in one HIP pass over the valid pairs
(mf_pair_mlp_bias) that builds the features from the adapters' tensors in registers and writes u, v, w in
the [B, H, N, N] layout with the diagonal and invalid pairs zero; the [B, N, N, hidden] activations of the
torch formulation never exist.  Other modes and CPU tensors take the torch formulation.
"""

from __future__ import annotations

from typing import Callable

import torch
import torch.nn.functional as F
from torch import nn

from matterformer_amd.geometry import GeometryFeatures
from matterformer_amd.simplicial_types import (
    SimplicialAttentionMask,
    SimplicialFactorizedBias,
    SimplicialLowRankAngleResidual,
    SimplicialLowRankMessageResidual,
)


def _softplus_inverse(value: torch.Tensor) -> torch.Tensor:
    """x with softplus(x) = value (transformer.py:31-33)."""
    v = value.clamp_min(1e-8)
    return v + torch.log(-torch.expm1(-v))


def build_simplicial_attention_mask(*, coords_len: int, seq_len: int, batch_size: int, device: torch.device,
                                    pad_mask: torch.Tensor | None = None,
                                    geom_pair_mask: torch.Tensor | None = None,
                                    include_global_tokens_as_pair_keys: bool = False) -> SimplicialAttentionMask:
    """Atom-only pair keys over the first coords_len tokens, the geometry pair mask as pair_valid
    (transformer.py:36-73)."""
    if seq_len < coords_len:
        raise ValueError(f"seq_len={seq_len} is smaller than coords_len={coords_len}")
    if pad_mask is None:
        query_valid = torch.ones(batch_size, seq_len, device=device, dtype=torch.bool)
    else:
        query_valid = ~pad_mask.bool().to(device=device)
    if include_global_tokens_as_pair_keys:
        return SimplicialAttentionMask(query_valid=query_valid, pair_key_valid=query_valid, pair_valid=None)
    is_atom = torch.arange(seq_len, device=device)[None, :] < coords_len
    pair_valid = None
    if geom_pair_mask is not None or seq_len != coords_len:
        pair_valid = torch.zeros(batch_size, seq_len, seq_len, device=device, dtype=torch.bool)
        atoms = True if geom_pair_mask is None else geom_pair_mask.bool().to(device=device)
        pair_valid[:, :coords_len, :coords_len] = atoms
    return SimplicialAttentionMask(query_valid=query_valid, pair_key_valid=query_valid & is_atom,
                                   pair_valid=pair_valid)


def _pair_mlp(hidden: int, out: int) -> nn.Sequential:
    return nn.Sequential(nn.LazyLinear(hidden), nn.SiLU(), nn.Linear(hidden, out))


class _GeometryBiasBase(nn.Module):
    """Noise gate and pair-bias helpers shared by the geometry bias modules (transformer.py:319-396)."""

    def __init__(self, n_heads: int, use_noise_gate: bool = True) -> None:
        super().__init__()
        self.n_heads = int(n_heads)
        self.use_noise_gate = bool(use_noise_gate)
        if self.use_noise_gate:
            ones = torch.ones((1, self.n_heads, 1, 1), dtype=torch.float32)
            self.noise_gate_alpha_raw = nn.Parameter(_softplus_inverse(ones))
            self.noise_gate_beta = nn.Parameter(torch.zeros((1, self.n_heads, 1, 1), dtype=torch.float32))

    @staticmethod
    def _mask_atom_pairwise_bias(pair_bias: torch.Tensor, atom_pad_mask: torch.Tensor | None) -> torch.Tensor:
        if atom_pad_mask is None:
            return pair_bias
        rows = atom_pad_mask[:, None, :, None]
        cols = atom_pad_mask[:, None, None, :]
        return pair_bias.masked_fill(rows, 0.0).masked_fill(cols, 0.0)

    @staticmethod
    def _zero_pairwise_diag(pair_bias: torch.Tensor) -> torch.Tensor:
        return pair_bias - torch.diag_embed(torch.diagonal(pair_bias, dim1=-2, dim2=-1))

    @staticmethod
    def _expand_atom_head_bias(bias_atoms: torch.Tensor, seq_len: int) -> torch.Tensor:
        B, H, n, _ = bias_atoms.shape
        if seq_len < n:
            raise ValueError(f"seq_len={seq_len} is smaller than the geometry length {n}")
        if seq_len == n:
            return bias_atoms
        full = bias_atoms.new_zeros(B, H, seq_len, seq_len)
        full[:, :, :n, :n] = bias_atoms
        return full

    def _sigma_gate(self, sigma: torch.Tensor | None, batch_size: int, dtype: torch.dtype,
                    device: torch.device) -> torch.Tensor:
        """(B, H, 1, 1): sigmoid(softplus(alpha_raw) * (-log sigma) + beta), or ones without the gate."""
        if not self.use_noise_gate:
            return torch.ones((batch_size, self.n_heads, 1, 1), device=device, dtype=dtype)
        if sigma is None:
            raise ValueError("sigma must be provided when use_noise_gate=True")
        if sigma.ndim == 2 and sigma.shape[1] == 1:
            sigma = sigma[:, 0]
        if sigma.ndim != 1:
            raise ValueError(f"sigma must have shape (B,) or (B, 1), got {tuple(sigma.shape)}")
        if sigma.shape[0] == 1 and batch_size > 1:
            sigma = sigma.expand(batch_size)
        if sigma.shape[0] != batch_size:
            raise ValueError(f"sigma batch {sigma.shape[0]} does not match batch size {batch_size}")
        noise_level = -torch.log(sigma.to(device=device, dtype=torch.float32).clamp_min(1e-8))
        alpha = F.softplus(self.noise_gate_alpha_raw).to(device=device, dtype=torch.float32)
        beta = self.noise_gate_beta.to(device=device, dtype=torch.float32)
        return torch.sigmoid(alpha * noise_level[:, None, None, None] + beta).to(dtype=dtype)


class SimplicialGeometryBias(_GeometryBiasBase):
    """The factorized bias u, v, w (+ low-rank angle / message factors) of simplicial attention from pair
    features (transformer.py:516-996)."""

    def __init__(self, n_heads: int, mode: str = "factorized", edge_bias_hidden_dim: int = 128,
                 edge_bias_n_rbf: int = 16, edge_bias_rbf_max: float = 2.0, edge_bias_n_freqs: int = 8,
                 angle_residual_rank: int = 16, message_mode: str = "none", message_rank: int = 16,
                 use_periodic_features: bool = False, use_noise_gate: bool = True) -> None:
        super().__init__(n_heads=n_heads, use_noise_gate=use_noise_gate)
        mode = mode.lower()
        if mode not in {"none", "factorized", "angle_residual", "angle_low_rank"}:
            raise ValueError(f"Unsupported simplicial geometry mode: {mode}")
        message_mode = message_mode.lower()
        if message_mode not in {"none", "low_rank"}:
            raise ValueError(f"Unsupported simplicial message mode: {message_mode}")
        self.mode = mode
        self.message_mode = message_mode
        self.use_periodic_features = bool(use_periodic_features)
        self.edge_bias_n_rbf = int(edge_bias_n_rbf)
        self.angle_residual_rank = int(angle_residual_rank)
        self.message_rank = int(message_rank)
        if self.angle_residual_rank <= 0:
            raise ValueError("angle_residual_rank must be positive")
        if self.message_mode == "low_rank" and self.message_rank <= 0:
            raise ValueError("message_rank must be positive when message_mode='low_rank'")
        self.register_buffer("_edge_rbf_centers",
                             torch.linspace(0.0, edge_bias_rbf_max, edge_bias_n_rbf, dtype=torch.float32),
                             persistent=False)
        spacing = edge_bias_rbf_max / max(edge_bias_n_rbf - 1, 1)
        self.register_buffer("_edge_rbf_gamma", torch.tensor(1.0 / max(spacing * spacing, 1e-6), dtype=torch.float32),
                             persistent=False)
        self._edge_rbf_gamma_value = float(self._edge_rbf_gamma)  # the same fp32 value, readable without a sync
        self.register_buffer("_edge_freqs", torch.arange(1, edge_bias_n_freqs + 1, dtype=torch.float32),
                             persistent=False)
        H, hidden = self.n_heads, edge_bias_hidden_dim
        # creation order of the reference module: u, v, w, angle residual, angle factors, message factors;
        # output layers start at zero except the right angle factor (zeroing both would stall its gradient)
        self.spoke_bias_u_mlp = self.spoke_bias_v_mlp = self.pair_bias_w_mlp = None
        if self.mode != "none":
            self.spoke_bias_u_mlp = _pair_mlp(hidden, H)
            self.spoke_bias_v_mlp = _pair_mlp(hidden, H)
            self.pair_bias_w_mlp = _pair_mlp(hidden, H)
            for mlp in (self.spoke_bias_u_mlp, self.spoke_bias_v_mlp, self.pair_bias_w_mlp):
                nn.init.zeros_(mlp[-1].weight)
                nn.init.zeros_(mlp[-1].bias)
        self.angle_residual_mlp = None
        if self.mode == "angle_residual":
            self.angle_residual_mlp = _pair_mlp(hidden, H)
            nn.init.zeros_(self.angle_residual_mlp[-1].weight)
            nn.init.zeros_(self.angle_residual_mlp[-1].bias)
        self.angle_left_mlp = self.angle_right_mlp = None
        if self.mode == "angle_low_rank":
            self.angle_left_mlp = _pair_mlp(hidden, H * self.angle_residual_rank)
            self.angle_right_mlp = _pair_mlp(hidden, H * self.angle_residual_rank)
            nn.init.zeros_(self.angle_left_mlp[-1].weight)
            nn.init.zeros_(self.angle_left_mlp[-1].bias)
        self.message_left_mlp = self.message_right_mlp = None
        if self.message_mode == "low_rank":
            self.message_left_mlp = _pair_mlp(hidden, H * self.message_rank)
            self.message_right_mlp = _pair_mlp(hidden, H * self.message_rank)
            nn.init.zeros_(self.message_left_mlp[-1].weight)
            nn.init.zeros_(self.message_left_mlp[-1].bias)

    # -- pair features (transformer.py:637-700) ----------------------------------------------------------------
    def _distance_rbf(self, dist_norm: torch.Tensor) -> torch.Tensor:
        centers = self._edge_rbf_centers.to(device=dist_norm.device, dtype=dist_norm.dtype)
        gamma = self._edge_rbf_gamma.to(device=dist_norm.device, dtype=dist_norm.dtype)
        return torch.exp(-gamma * (dist_norm.unsqueeze(-1) - centers.view(1, 1, 1, -1)).square())

    def _periodic_terms(self, g: GeometryFeatures, with_fourier: bool) -> list[torch.Tensor]:
        if not (self.use_periodic_features and g.kind == "periodic"):
            return []
        B, n = g.pair_delta.shape[:2]
        terms = []
        if with_fourier:
            freqs = self._edge_freqs.to(device=g.pair_delta.device, dtype=g.pair_delta.dtype)
            phase = 2.0 * torch.pi * g.pair_delta[..., None] * freqs.view(1, 1, 1, 1, -1)
            terms.append(torch.cat([torch.sin(phase), torch.cos(phase)], dim=-1).reshape(B, n, n, -1))
        terms.append(g.global_geom[:, None, None, :].expand(-1, n, n, -1))
        return terms

    def _build_spoke_features(self, geom_features: GeometryFeatures) -> torch.Tensor:
        g = geom_features
        return torch.cat([g.pair_delta, self._distance_rbf(g.pair_dist_norm)] + self._periodic_terms(g, True), dim=-1)

    def _build_angle_spoke_features(self, geom_features: GeometryFeatures) -> torch.Tensor:
        g = geom_features
        inv_d = g.pair_dist.clamp_min(1e-8).unsqueeze(-1)
        keep = g.pair_mask.unsqueeze(-1)
        unit = torch.where(keep, g.pair_delta / inv_d, torch.zeros_like(g.pair_delta))
        metric = g.extras["metric"].to(device=g.pair_delta.device, dtype=g.pair_delta.dtype)
        metric_unit = torch.einsum("bnmd,bdc->bnmc", g.pair_delta, metric) / inv_d
        metric_unit = torch.where(keep, metric_unit, torch.zeros_like(metric_unit))
        parts = [unit, metric_unit, g.pair_delta, self._distance_rbf(g.pair_dist_norm)]
        return torch.cat(parts + self._periodic_terms(g, True), dim=-1)

    def _build_pair_features(self, geom_features: GeometryFeatures) -> torch.Tensor:
        g = geom_features
        return torch.cat([self._distance_rbf(g.pair_dist_norm)] + self._periodic_terms(g, False), dim=-1)

    # -- terms (transformer.py:702-750) ------------------------------------------------------------------------
    def _compute_factorized_terms(self, geom_features: GeometryFeatures):
        if self.spoke_bias_u_mlp is None or self.spoke_bias_v_mlp is None or self.pair_bias_w_mlp is None:
            raise RuntimeError("Factorized simplicial geometry requested without factorized geometry MLPs")
        from matterformer_amd import pair_mlp

        if pair_mlp.serves(self, geom_features):
            return pair_mlp.factorized_terms(self, geom_features)
        spoke = self._build_spoke_features(geom_features)
        pair = self._build_pair_features(geom_features)
        terms = [mlp(feat).permute(0, 3, 1, 2).contiguous()
                 for mlp, feat in ((self.spoke_bias_u_mlp, spoke), (self.spoke_bias_v_mlp, spoke),
                                   (self.pair_bias_w_mlp, pair))]
        mask = geom_features.pair_mask[:, None, :, :].to(dtype=terms[0].dtype)
        return tuple(self._zero_pairwise_diag(t) * mask for t in terms)

    def _low_rank_factors(self, geom_features: GeometryFeatures, left_mlp: nn.Module, right_mlp: nn.Module,
                          rank: int):
        feats = self._build_angle_spoke_features(geom_features)
        B, n = geom_features.pair_delta.shape[:2]
        shape = (B, n, n, self.n_heads, rank)
        pair_mask = geom_features.pair_mask[:, None, :, :, None].to(dtype=feats.dtype)
        eye = torch.eye(n, device=feats.device, dtype=torch.bool).view(1, 1, n, n, 1)
        out = []
        for mlp in (left_mlp, right_mlp):
            f = mlp(feats).view(shape).permute(0, 3, 1, 2, 4).contiguous()
            out.append(f.masked_fill(eye, 0.0) * pair_mask)
        return tuple(out)

    def _compute_low_rank_angle_residual(self, geom_features: GeometryFeatures):
        if self.angle_left_mlp is None or self.angle_right_mlp is None:
            raise RuntimeError("Low-rank angle residual requested without low-rank angle MLPs")
        return self._low_rank_factors(geom_features, self.angle_left_mlp, self.angle_right_mlp,
                                      self.angle_residual_rank)

    def _compute_low_rank_message_residual(self, geom_features: GeometryFeatures):
        if self.message_left_mlp is None or self.message_right_mlp is None:
            raise RuntimeError("Low-rank message residual requested without message MLPs")
        return self._low_rank_factors(geom_features, self.message_left_mlp, self.message_right_mlp,
                                      self.message_rank)

    @staticmethod
    def _mask_atom_pairwise_rank_factor(factor: torch.Tensor, atom_pad_mask: torch.Tensor | None) -> torch.Tensor:
        if atom_pad_mask is None:
            return factor
        return factor.masked_fill(atom_pad_mask[:, None, :, None, None], 0.0).masked_fill(
            atom_pad_mask[:, None, None, :, None], 0.0)

    @staticmethod
    def _expand_atom_head_rank_factor(factor_atoms: torch.Tensor, seq_len: int) -> torch.Tensor:
        B, H, n, _, R = factor_atoms.shape
        if seq_len < n:
            raise ValueError(f"seq_len={seq_len} is smaller than the geometry length {n}")
        if seq_len == n:
            return factor_atoms
        full = factor_atoms.new_zeros(B, H, seq_len, seq_len, R)
        full[:, :, :n, :n, :] = factor_atoms
        return full

    def _compute_angle_residual_chunk(self, geom_features: GeometryFeatures, q_start: int, q_end: int):
        """Dense angle residual of queries q_start..q_end (transformer.py:788-818)."""
        if self.angle_residual_mlp is None:
            raise RuntimeError("Angle residual requested without angle_residual_mlp")
        g = geom_features
        dq = g.pair_delta[:, q_start:q_end]
        dist = g.pair_dist[:, q_start:q_end]
        metric = g.extras["metric"].to(device=dq.device, dtype=dq.dtype)
        num = torch.einsum("bqjc,bqkc->bqjk", torch.einsum("bqnd,bdc->bqnc", dq, metric), dq)
        den = dist[:, :, :, None] * dist[:, :, None, :]
        pm = g.pair_mask[:, q_start:q_end]
        valid = (den > 1e-8) & pm[:, :, :, None] & pm[:, :, None, :]
        cos = torch.where(valid, num / den.clamp_min(1e-8), torch.zeros_like(num)).clamp(min=-1.0, max=1.0)
        rbf = self._distance_rbf(g.pair_dist_norm[:, q_start:q_end])
        n = rbf.shape[2]
        tri = torch.cat([rbf.unsqueeze(-2).expand(-1, -1, -1, n, -1), rbf.unsqueeze(-3).expand(-1, -1, n, -1, -1),
                         cos.unsqueeze(-1)], dim=-1)
        out = self.angle_residual_mlp(tri).permute(0, 4, 1, 2, 3).contiguous()
        return out * valid[:, None].to(dtype=out.dtype)

    # -- assembly (transformer.py:820-995) ---------------------------------------------------------------------
    def build_structured_bias_inputs(self, geom_features: GeometryFeatures, coords_len: int,
                                     pad_mask: torch.Tensor | None = None, seq_len: int | None = None,
                                     sigma: torch.Tensor | None = None):
        """(factorized_bias, logit_bias_fn, angle_residual, message_residual, attention_mask)."""
        atom_pad = pad_mask[:, :coords_len].bool() if pad_mask is not None else None
        T = seq_len or coords_len
        src = geom_features.pair_dist_norm
        gate = self._sigma_gate(sigma=sigma, batch_size=src.shape[0], dtype=src.dtype, device=src.device)
        gate = gate.expand(-1, -1, T, -1).squeeze(-1)
        if T > coords_len:
            gate = gate * (torch.arange(T, device=gate.device) < coords_len).to(dtype=gate.dtype).view(1, 1, T)
        attention_mask = build_simplicial_attention_mask(coords_len=coords_len, seq_len=T, batch_size=gate.shape[0],
                                                         device=gate.device, pad_mask=pad_mask,
                                                         geom_pair_mask=geom_features.pair_mask)

        def pair_terms(parts):
            return [self._expand_atom_head_bias(self._mask_atom_pairwise_bias(t, atom_pad), seq_len=T) for t in parts]

        def rank_terms(parts):
            return [self._expand_atom_head_rank_factor(self._mask_atom_pairwise_rank_factor(t, atom_pad), seq_len=T)
                    for t in parts]

        factorized = None
        if self.mode != "none":
            u, v, w = pair_terms(self._compute_factorized_terms(geom_features))
            factorized = SimplicialFactorizedBias(u=u, v=v, w=w, gate=gate)
        message = None
        if self.message_mode == "low_rank":
            left, right = rank_terms(self._compute_low_rank_message_residual(geom_features))
            message = SimplicialLowRankMessageResidual(left=left, right=right)
        if self.mode == "none":
            return None, None, None, message, attention_mask
        if self.mode == "factorized":
            return factorized, None, None, message, attention_mask
        if self.mode == "angle_low_rank":
            left, right = rank_terms(self._compute_low_rank_angle_residual(geom_features))
            angle = SimplicialLowRankAngleResidual(left=left, right=right, gate=gate)
            return factorized, None, angle, message, attention_mask

        def residual_fn(start: int, end: int, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
            res = torch.zeros(gate.shape[0], self.n_heads, end - start, T, T, device=gate.device, dtype=gate.dtype)
            stop = min(end, coords_len)
            if start < stop:
                res[:, :, : stop - start, :coords_len, :coords_len] = self._compute_angle_residual_chunk(
                    geom_features, start, stop)
            return (gate[:, :, start:end, None, None] * res).to(device=device, dtype=dtype)

        return factorized, residual_fn, None, message, attention_mask

    def build_bias_inputs(self, geom_features: GeometryFeatures, coords_len: int, pad_mask: torch.Tensor | None = None,
                          seq_len: int | None = None, sigma: torch.Tensor | None = None):
        """(factorized_bias, logit_bias_fn, attention_mask), the low-rank angle folded into the callback."""
        factorized, residual_fn, angle, _, mask = self.build_structured_bias_inputs(
            geom_features=geom_features, coords_len=coords_len, pad_mask=pad_mask, seq_len=seq_len, sigma=sigma)
        if residual_fn is None and angle is not None:
            def residual_fn(start, end, dtype, device):
                return angle.chunk(start, end, dtype=dtype, device=device)
        return factorized, residual_fn, mask

    def build_logit_bias_fn(self, geom_features: GeometryFeatures, coords_len: int,
                            pad_mask: torch.Tensor | None = None, seq_len: int | None = None,
                            sigma: torch.Tensor | None = None) -> Callable[[int, int, torch.dtype, torch.device],
                                                                          torch.Tensor]:
        """One callback with every logit term (factorized bias + angle) for the torch path."""
        factorized, residual_fn, angle, _, _ = self.build_structured_bias_inputs(
            geom_features=geom_features, coords_len=coords_len, pad_mask=pad_mask, seq_len=seq_len, sigma=sigma)

        def bias_fn(start: int, end: int, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
            if factorized is None:
                raise RuntimeError("build_logit_bias_fn requires a non-none simplicial geometry mode")
            bias = factorized.chunk(start, end, dtype=dtype, device=device)
            if residual_fn is not None:
                return bias + residual_fn(start, end, dtype, device)
            if angle is not None:
                return bias + angle.chunk(start, end, dtype=dtype, device=device)
            return bias

        return bias_fn
