"""Alternating 2-simplicial / kNN-local AdaLN trunk.

Blocks mirror the reference's AdaLNBlock (src/matterformer/models/transformer.py:154-316) and Mlp
(:129-148): the same submodules, created in the same order with the same classes and names, so a
seeded construction draws the reference's initial weights and a reference block's state dict loads.
The reference trunk has one global attn_type (transformer.py:1150-1177) and no kNN attention; the
configs[4] trunk alternates

  even blocks  attn_type="simplicial": SimplicialAttention (the HIP kernels behind the reference API)
  odd blocks   attn_type="knn_local": multi-head attention of every atom over its k nearest
               neighbours and itself -- the reference's attn_type="mha" block with a 0 / -inf
               attn_head_bias (transformer.py:256-268) -- with nn.MultiheadAttention's parameters
               (attn.attn.in_proj_weight, ...); on the GPU: in_proj, mf_radius_attn over the kNN bit
               mask (mf_knn -> mf_knn_mask), out_proj.

The kNN lists and masks are built once per forward from the coordinates and shared by the local blocks.
impl="auto" runs the HIP kernels for GPU tensors (a missing library raises) and the reference's own
torch modules for CPU tensors; impl="torch" forces the latter.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from matterformer_amd.simplicial_attention import SimplicialAttention
from matterformer_amd.simplicial_types import SimplicialAttentionMask

ATTN_TYPES = ("simplicial", "knn_local")


def _modulate(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    return x * (1.0 + scale[:, None, :]) + shift[:, None, :]


class Mlp(nn.Module):
    """fc1 -> tanh-GELU -> fc2 (transformer.py:129-148)."""

    def __init__(self, d_model: int, mlp_ratio: float = 4.0, dropout: float = 0.0) -> None:
        super().__init__()
        hidden = int(d_model * mlp_ratio)
        self.fc1 = nn.Linear(d_model, hidden)
        self.act = nn.GELU(approximate="tanh")
        self.drop1 = nn.Dropout(dropout)
        self.fc2 = nn.Linear(hidden, d_model)
        self.drop2 = nn.Dropout(dropout)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.drop2(self.fc2(self.drop1(self.act(self.fc1(x)))))


def knn_lists_torch(coords: torch.Tensor, k: int, pad_mask: torch.Tensor | None) -> torch.Tensor:
    """kNN lists by the mf_knn convention, in torch: d2 = (dx^2 + dy^2) + dz^2 in fp32, ascending (d2, j),
    self and padded atoms excluded, -1 past the last candidate and for padded atoms.  The impl="torch" path."""
    B, N, _ = coords.shape
    c = coords.float()
    d = c[:, :, None, :] - c[:, None, :, :]
    d2 = (d[..., 0] * d[..., 0] + d[..., 1] * d[..., 1]) + d[..., 2] * d[..., 2]
    bad = torch.eye(N, dtype=torch.bool, device=c.device)[None].expand(B, N, N).clone()
    if pad_mask is not None:
        bad |= pad_mask[:, None, :].bool() | pad_mask[:, :, None].bool()
    d2 = d2.masked_fill(bad, float("inf"))
    order = torch.sort(d2, dim=-1, stable=True)
    kk = min(k, N)
    idx = order.indices[..., :kk].to(torch.int32)
    idx = torch.where(torch.isinf(order.values[..., :kk]), torch.full_like(idx, -1), idx)
    if kk < k:
        idx = torch.cat([idx, torch.full((B, N, k - kk), -1, dtype=torch.int32, device=c.device)], dim=-1)
    return idx


def knn_allowed_torch(idx: torch.Tensor, pad_mask: torch.Tensor | None) -> torch.Tensor:
    """(B, N, N) bool: j in idx[i] or j == i, for valid i (the bits mf_knn_mask writes)."""
    B, N, K = idx.shape
    allowed = torch.zeros(B, N, N + 1, dtype=torch.bool, device=idx.device)
    cols = torch.where(idx < 0, torch.full_like(idx, N), idx).long()
    allowed.scatter_(2, cols, True)
    allowed = allowed[..., :N] | torch.eye(N, dtype=torch.bool, device=idx.device)[None]
    if pad_mask is not None:
        allowed &= ~pad_mask.bool()[:, :, None]
    return allowed


class KnnLocalMask:
    """The local blocks' mask, built once per forward: kNN lists plus bit / block masks (GPU) or the
    boolean matrix (CPU)."""

    def __init__(self, idx: torch.Tensor, bits=None, blocks=None, allowed=None):
        self.idx = idx
        self.bits = bits
        self.blocks = blocks
        self.allowed = allowed


def build_knn_mask(coords: torch.Tensor, k: int, pad_mask: torch.Tensor | None, *, use_hip: bool) -> KnnLocalMask:
    if use_hip:
        from matterformer_amd.geometry_ops import knn_graph, knn_mask

        idx = knn_graph(coords, k, pad_mask, exclude_self=True, return_dist=False)
        bits, blocks = knn_mask(idx, pad_mask, include_self=True)
        return KnnLocalMask(idx, bits=bits, blocks=blocks)
    idx = knn_lists_torch(coords, k, pad_mask)
    return KnnLocalMask(idx, allowed=knn_allowed_torch(idx, pad_mask))


class KnnLocalAttention(nn.Module):
    """MHA of every atom over its kNN mask.  Parameters are nn.MultiheadAttention's, held as ``attn``
    like the reference's RegularAttention (regular_attention.py:275-338), so state dicts match."""

    def __init__(self, d_model: int, n_heads: int, *, dropout: float = 0.0, impl: str = "auto") -> None:
        super().__init__()
        impl = impl.lower()
        if impl == "hip":
            impl = "triton"
        if impl not in {"auto", "torch", "triton"}:
            raise ValueError(f"Unsupported local attention impl: {impl}")
        self.impl = impl
        self.attn = nn.MultiheadAttention(d_model, n_heads, dropout=dropout, batch_first=True)
        self._last_impl_used = "torch"

    def _use_hip(self, h: torch.Tensor) -> bool:
        if self.impl == "torch" or h.device.type != "cuda":
            if self.impl == "triton":
                raise RuntimeError("the HIP local attention requires GPU tensors")
            return False
        if self.training and self.attn.dropout > 0.0:
            if self.impl == "triton":
                raise RuntimeError("the HIP local attention does not support attention dropout in training mode")
            return False
        return True

    def forward(self, h: torch.Tensor, mask: KnnLocalMask, pad_mask: torch.Tensor | None = None) -> torch.Tensor:
        if self._use_hip(h):
            from matterformer_amd.geometry_ops import radius_attention

            if mask.bits is None:
                raise RuntimeError("the HIP local attention needs the kNN bit mask (build_knn_mask(use_hip=True))")
            self._last_impl_used = "triton"
            mha = self.attn
            B, T, C = h.shape
            H = mha.num_heads
            D = C // H
            qkv = F.linear(h, mha.in_proj_weight, mha.in_proj_bias)
            cdt = h.dtype if h.dtype in (torch.bfloat16, torch.float16) else torch.bfloat16
            q, k, v = (t.reshape(B, T, H, D).transpose(1, 2).to(cdt).contiguous() for t in qkv.chunk(3, dim=-1))
            out = radius_attention(q, k, v, mask.bits, mask.blocks, scale=D ** -0.5)
            out = out.transpose(1, 2).reshape(B, T, C).to(h.dtype)
            return F.linear(out, mha.out_proj.weight, mha.out_proj.bias)
        self._last_impl_used = "torch"
        allowed = mask.allowed if mask.allowed is not None else knn_allowed_torch(mask.idx, pad_mask)
        B, T, _ = h.shape
        H = self.attn.num_heads
        # the reference's attn_head_bias route (transformer.py:256-268): 0 / -inf, padded keys at finfo.min;
        # a padded query keeps itself so its softmax row is defined (its output is never read by valid rows)
        allowed = allowed | torch.eye(T, dtype=torch.bool, device=h.device)[None]
        bias = torch.zeros(B, T, T, dtype=h.dtype, device=h.device).masked_fill(~allowed, float("-inf"))
        attn_mask = bias[:, None].expand(B, H, T, T).reshape(B * H, T, T)
        kpm = None
        if pad_mask is not None:
            kpm = torch.zeros(B, T, dtype=h.dtype, device=h.device).masked_fill(pad_mask.bool(),
                                                                                 torch.finfo(h.dtype).min)
        out, _ = self.attn(h, h, h, key_padding_mask=kpm, need_weights=False, attn_mask=attn_mask)
        return out


class AdaLNBlock(nn.Module):
    """Pre-norm block with adaLN modulation (transformer.py:154-316) for attn_type in ATTN_TYPES."""

    def __init__(
        self,
        d_model: int,
        n_heads: int,
        mlp_ratio: float = 4.0,
        dropout: float = 0.0,
        attn_dropout: float = 0.0,
        eps: float = 1e-6,
        attn_type: str = "simplicial",
        simplicial_chunk_size: int = 128,
        simplicial_head_dim: int | None = None,
        simplicial_impl: str = "auto",
        simplicial_precision: str = "bf16_tc",
        simplicial_message_mode: str = "none",
        simplicial_message_rank: int = 16,
        simplicial_content_logits: str = "on",
        local_impl: str = "auto",
        use_adaln_conditioning: bool = True,
        norm_affine_when_no_adaln: bool = False,
    ) -> None:
        super().__init__()
        attn_type = attn_type.lower()
        if attn_type not in ATTN_TYPES:
            raise ValueError(f"Unsupported attn_type: {attn_type}; expected one of {ATTN_TYPES}")
        self.attn_type = attn_type
        self.n_heads = int(n_heads)
        self.use_adaln_conditioning = bool(use_adaln_conditioning)
        norm_affine = bool(norm_affine_when_no_adaln) and not self.use_adaln_conditioning
        # creation order of the reference block: norms, ada_ln, attention, mlp
        self.norm1 = nn.LayerNorm(d_model, eps=eps, elementwise_affine=norm_affine)
        self.norm2 = nn.LayerNorm(d_model, eps=eps, elementwise_affine=norm_affine)
        if self.use_adaln_conditioning:
            self.ada_ln = nn.Sequential(nn.SiLU(), nn.Linear(d_model, 6 * d_model, bias=True))
            nn.init.zeros_(self.ada_ln[-1].weight)
            nn.init.zeros_(self.ada_ln[-1].bias)
        else:
            self.ada_ln = None
        if attn_type == "knn_local":
            self.attn = KnnLocalAttention(d_model, self.n_heads, dropout=attn_dropout, impl=local_impl)
        else:
            self.attn = SimplicialAttention(
                dim=d_model, num_heads=self.n_heads, head_dim=simplicial_head_dim, dropout=attn_dropout,
                chunk_size=simplicial_chunk_size, bias=True, out_proj=True, impl=simplicial_impl,
                precision=simplicial_precision, message_mode=simplicial_message_mode,
                message_rank=simplicial_message_rank, content_logits=simplicial_content_logits)
        self.mlp = Mlp(d_model=d_model, mlp_ratio=mlp_ratio, dropout=dropout)

    def forward(self, x: torch.Tensor, cond_emb: torch.Tensor | None, pad_mask: torch.Tensor | None = None, *,
                knn_mask: KnnLocalMask | None = None,
                simplicial_attention_mask: SimplicialAttentionMask | None = None,
                simplicial_factorized_bias=None) -> torch.Tensor:
        if self.use_adaln_conditioning:
            if cond_emb is None or cond_emb.ndim != 2 or cond_emb.shape[-1] != x.shape[-1]:
                raise ValueError(f"cond_emb must have shape (B, {x.shape[-1]})")
            shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = self.ada_ln(cond_emb).chunk(6, dim=-1)
            h = _modulate(self.norm1(x), shift_msa, scale_msa)
        else:
            h = self.norm1(x)
        if self.attn_type == "knn_local":
            if knn_mask is None:
                raise ValueError("a knn_local block needs knn_mask")
            attn_out = self.attn(h, knn_mask, pad_mask)
        else:
            attn_out = self.attn(h, key_padding_mask=pad_mask, attention_mask=simplicial_attention_mask,
                                 factorized_bias=simplicial_factorized_bias)
        if self.use_adaln_conditioning:
            x = x + gate_msa[:, None, :] * attn_out
            h = _modulate(self.norm2(x), shift_mlp, scale_mlp)
            return x + gate_mlp[:, None, :] * self.mlp(h)
        x = x + attn_out
        return x + self.mlp(self.norm2(x))


class AlternatingTrunk(nn.Module):
    """n_layers AdaLN blocks, simplicial on even and kNN-local (k = knn_k) on odd layers by default."""

    def __init__(self, d_model: int = 512, n_heads: int = 8, n_layers: int = 12, *, mlp_ratio: float = 4.0,
                 knn_k: int = 32, schedule: list[str] | None = None, simplicial_impl: str = "auto",
                 simplicial_precision: str = "bf16_tc", local_impl: str = "auto", eps: float = 1e-6,
                 use_adaln_conditioning: bool = True) -> None:
        super().__init__()
        if schedule is None:
            schedule = ["simplicial" if layer % 2 == 0 else "knn_local" for layer in range(n_layers)]
        if len(schedule) != n_layers:
            raise ValueError("schedule must name one attention type per layer")
        self.knn_k = int(knn_k)
        self.schedule = list(schedule)
        self.blocks = nn.ModuleList([
            AdaLNBlock(d_model, n_heads, mlp_ratio=mlp_ratio, eps=eps, attn_type=t, simplicial_impl=simplicial_impl,
                       simplicial_precision=simplicial_precision, local_impl=local_impl,
                       use_adaln_conditioning=use_adaln_conditioning)
            for t in self.schedule])

    def _use_hip(self, x: torch.Tensor) -> bool:
        local = [b.attn for b in self.blocks if b.attn_type == "knn_local"]
        return x.device.type == "cuda" and any(a.impl != "torch" for a in local)

    def forward(self, x: torch.Tensor, cond_emb: torch.Tensor | None, coords: torch.Tensor,
                pad_mask: torch.Tensor | None = None) -> torch.Tensor:
        mask = None
        if "knn_local" in self.schedule:
            mask = build_knn_mask(coords, self.knn_k, pad_mask, use_hip=self._use_hip(x))
        for block in self.blocks:
            x = block(x, cond_emb, pad_mask, knn_mask=mask)
        return x
