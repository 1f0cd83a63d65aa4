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

Like the reference's TransformerTrunk (transformer.py:1298-1316) the trunk zeroes padded atoms before every
block and in its output.  Every valid row's result is independent of the padded rows (attention masks padded
keys; everything else is per token), so on the GPU the trunk runs packed (``TokenPacking``): the per-token
work -- LayerNorm, modulation, the linears, the MLP, the residuals -- runs on the valid atoms only, as one
(T, C) matrix, and only the attention cores see the padded (B, H, N, D) layout their kernels read, which the
packed projections are scattered into (padded rows zero) and gathered back from.  On GEOM-Drugs batches
(about 44 atoms padded to 181) that removes about three quarters of the linear-layer work.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from matterformer_amd.simplicial_attention import SimplicialAttention
from matterformer_amd.simplicial_types import SimplicialAttentionMask, coerce_attention_mask
from matterformer_amd.token_packing import TokenPacking, adaln_rows

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
        if self._fused_gelu_ok(x):
            # fc1 with the tanh-GELU in the GEMM epilogue (hipBLASLt), applied to the fp32 accumulator
            h = torch._addmm_activation(self.fc1.bias, x, self.fc1.weight.t(), use_gelu=True)
            return self.fc2(h)
        return self.drop2(self.fc2(self.drop1(self.act(self.fc1(x)))))

    def _fused_gelu_ok(self, x: torch.Tensor) -> bool:
        """Inference on packed GPU rows: a 2-D input, dropout inactive, no autograd through the call."""
        if x.device.type != "cuda" or x.ndim != 2 or self.fc1.bias is None:
            return False
        if self.training and (self.drop1.p > 0.0 or self.drop2.p > 0.0):
            return False
        return not (torch.is_grad_enabled() and (x.requires_grad or self.fc1.weight.requires_grad))


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

    def _hip_unavailable_reason(self, h: torch.Tensor) -> str | None:
        if h.device.type != "cuda":
            return "the HIP local attention requires GPU tensors"
        if self.training and self.attn.dropout > 0.0:
            return "the HIP local attention does not support attention dropout in training mode"
        if torch.is_grad_enabled() and (h.requires_grad or any(p.requires_grad for p in self.attn.parameters())):
            # mf_radius_attn is a forward kernel with no autograd Function: the torch path keeps the graph
            return "the HIP local attention has no backward; autograd takes the torch path"
        head_dim = self.attn.embed_dim // self.attn.num_heads
        if head_dim not in (32, 64, 128):
            return f"the HIP local attention supports head_dim 32, 64 or 128, got {head_dim}"
        return None

    def _use_hip(self, h: torch.Tensor) -> bool:
        if self.impl == "torch":
            return False
        reason = self._hip_unavailable_reason(h)
        if reason is not None and self.impl == "triton":
            raise RuntimeError(reason)
        return reason is None

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
        return self._forward_torch(h, mask, pad_mask)

    def forward_packed(self, hp: torch.Tensor, mask: KnnLocalMask, packing: TokenPacking) -> torch.Tensor:
        """The HIP path on packed rows: in_proj on (T, C), the kernel over the padded head layout, out_proj."""
        if not self._use_hip(hp):
            raise RuntimeError("packed local attention runs on the HIP kernels only")
        if mask.bits is None:
            raise RuntimeError("the HIP local attention needs the kNN bit mask (build_knn_mask(use_hip=True))")
        from matterformer_amd.geometry_ops import radius_attention

        self._last_impl_used = "triton"
        mha = self.attn
        H = mha.num_heads
        D = hp.shape[-1] // H
        cdt = hp.dtype if hp.dtype in (torch.bfloat16, torch.float16) else torch.bfloat16
        qkv = packing.to_heads(F.linear(hp, mha.in_proj_weight, mha.in_proj_bias), 3, H, D, cdt)
        out = radius_attention(qkv[0], qkv[1], qkv[2], mask.bits, mask.blocks, scale=D ** -0.5)
        return F.linear(packing.from_heads(out, hp.dtype), mha.out_proj.weight, mha.out_proj.bias)

    def _forward_torch(self, h: torch.Tensor, mask: KnnLocalMask, pad_mask: torch.Tensor | None) -> torch.Tensor:
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


class SimplicialTerms:
    """The simplicial blocks' shared inputs: attention mask and the optional logit / message terms (the
    reference trunk builds them once per forward, transformer.py:1261-1296)."""

    def __init__(self, attention_mask: SimplicialAttentionMask | None, factorized_bias=None, angle_residual=None,
                 message_residual=None, logit_bias_fn=None) -> None:
        self.attention_mask = attention_mask
        self.factorized_bias = factorized_bias
        self.angle_residual = angle_residual
        self.message_residual = message_residual
        self.logit_bias_fn = logit_bias_fn

    def block_kwargs(self) -> dict:
        return dict(simplicial_attention_mask=self.attention_mask, simplicial_factorized_bias=self.factorized_bias,
                    simplicial_angle_residual=self.angle_residual, simplicial_message_residual=self.message_residual,
                    simplicial_logit_bias_fn=self.logit_bias_fn)

    def compact(self, packing: TokenPacking) -> "SimplicialTerms":
        """Every term in the packing's compact layout (atom axes N -> W)."""
        if self.logit_bias_fn is not None:
            raise RuntimeError("a dense logit_bias_fn cannot be packed")
        from matterformer_amd.simplicial_types import (SimplicialFactorizedBias, SimplicialLowRankAngleResidual,
                                                       SimplicialLowRankMessageResidual)

        c = packing.compact_dims
        m = self.attention_mask
        mask = SimplicialAttentionMask(query_valid=c(m.query_valid, 1), pair_key_valid=c(m.pair_key_valid, 1),
                                       pair_valid=None if m.pair_valid is None else c(m.pair_valid, 1, 2))
        fb = self.factorized_bias
        if fb is not None:
            fb = SimplicialFactorizedBias(u=c(fb.u, 2, 3), v=c(fb.v, 2, 3), w=c(fb.w, 2, 3), gate=c(fb.gate, 2))
        ang = self.angle_residual
        if ang is not None:
            ang = SimplicialLowRankAngleResidual(left=c(ang.left, 2, 3), right=c(ang.right, 2, 3), gate=c(ang.gate, 2))
        msg = self.message_residual
        if msg is not None:
            msg = SimplicialLowRankMessageResidual(left=c(msg.left, 2, 3), right=c(msg.right, 2, 3))
        return SimplicialTerms(mask, fb, ang, msg)


def _simplicial_packed(attn: SimplicialAttention, hp: torch.Tensor, packing: TokenPacking,
                       terms: SimplicialTerms) -> torch.Tensor:
    """SimplicialAttention.forward's HIP branch on packed rows: in_proj and out_proj on (T, C); q scaled and
    content-gated in the projection dtype as in _project_inputs / _content_query; the core on the padded
    head layout."""
    attn._last_impl_used = "triton"
    on = attn.content_logits == "on"
    # the kernels read the compute dtype; q's scale is applied (and rounded) in the projection dtype first
    dtype = attn._triton_compute_dtype() if on else hp.dtype
    parts = packing.to_heads(attn.in_proj(hp), 5, attn.num_heads, attn.head_dim, dtype,
                             first_part_scale=attn.scale)
    q = parts[0] if on else attn._content_query(parts[0])
    msg = terms.message_residual
    out = attn._forward_triton(q, parts[1], parts[2], parts[3], parts[4], attention_mask=terms.attention_mask,
                               factorized_bias=terms.factorized_bias, angle_residual=terms.angle_residual,
                               message_residual=msg, message_basis=attn.message_basis if msg is not None else None)
    return attn.out_proj(packing.from_heads(out, hp.dtype))


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
                simplicial_factorized_bias=None, simplicial_angle_residual=None, simplicial_message_residual=None,
                simplicial_logit_bias_fn=None) -> torch.Tensor:
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
                                 factorized_bias=simplicial_factorized_bias, angle_residual=simplicial_angle_residual,
                                 message_residual=simplicial_message_residual, logit_bias_fn=simplicial_logit_bias_fn)
        if self.use_adaln_conditioning:
            x = x + gate_msa[:, None, :] * attn_out
            h = _modulate(self.norm2(x), shift_mlp, scale_mlp)
            return x + gate_mlp[:, None, :] * self.mlp(h)
        x = x + attn_out
        return x + self.mlp(self.norm2(x))

    def _mods(self, cond_emb: torch.Tensor | None, batch: int) -> torch.Tensor:
        """ada_ln(cond_emb) as (B, 6C): shift, scale, gate of the attention half, then of the MLP half."""
        if cond_emb is None or cond_emb.ndim != 2 or cond_emb.shape[0] != batch:
            raise ValueError("cond_emb must have shape (B, C)")
        return self.ada_ln(cond_emb).contiguous()

    def _attention_packed(self, h: torch.Tensor, packing: TokenPacking, knn_mask: KnnLocalMask | None,
                          terms: "SimplicialTerms | None") -> torch.Tensor:
        if self.attn_type == "knn_local":
            if knn_mask is None:
                raise ValueError("a knn_local block needs knn_mask")
            return self.attn.forward_packed(h, knn_mask, packing)
        if terms is None or terms.attention_mask is None:
            raise ValueError("a packed simplicial block needs the attention mask of the compact batch")
        return _simplicial_packed(self.attn, h, packing, terms)

    def forward_packed(self, xp: torch.Tensor, cond_emb: torch.Tensor | None, packing: TokenPacking, *,
                       knn_mask: KnnLocalMask | None = None, terms: "SimplicialTerms | None" = None) -> torch.Tensor:
        """forward on the valid rows (T, C) of a batch (TokenPacking); masks and simplicial terms in the packing's
        compact layout.  The same operations in the same dtypes as forward."""
        if not self.use_adaln_conditioning:
            h = self.norm1(xp)
            xp = xp + self._attention_packed(h, packing, knn_mask, terms)
            return xp + self.mlp(self.norm2(xp))
        C = xp.shape[-1]
        mods = self._mods(cond_emb, packing.batch)
        h = adaln_rows(packing, xp, shift=mods[:, :C], scale=mods[:, C:2 * C], eps=self.norm1.eps)
        a = self._attention_packed(h, packing, knn_mask, terms)
        xp, h = adaln_rows(packing, xp, a, gate=mods[:, 2 * C:3 * C], shift=mods[:, 3 * C:4 * C],
                           scale=mods[:, 4 * C:5 * C], eps=self.norm2.eps)
        return adaln_rows(packing, xp, self.mlp(h), gate=mods[:, 5 * C:])


class AlternatingTrunk(nn.Module):
    """n_layers AdaLN blocks, simplicial on even and kNN-local (k = knn_k) on odd layers by default."""

    def __init__(self, d_model: int = 512, n_heads: int = 8, n_layers: int = 12, *, mlp_ratio: float = 4.0,
                 knn_k: int = 32, schedule: list[str] | None = None, simplicial_impl: str = "auto",
                 simplicial_precision: str = "bf16_tc", simplicial_message_mode: str = "none",
                 simplicial_message_rank: int = 16, simplicial_content_logits: str = "on", local_impl: str = "auto",
                 eps: float = 1e-6, use_adaln_conditioning: bool = True, geometry_adapter: nn.Module | None = None,
                 simplicial_geometry_bias: nn.Module | None = None, pack_tokens: bool = True) -> None:
        super().__init__()
        self.pack_tokens = bool(pack_tokens)
        # registered before the blocks, as in TransformerTrunk.__init__ (transformer.py:1137-1139)
        self.geometry_adapter = geometry_adapter
        self.simplicial_geometry_bias = simplicial_geometry_bias
        if schedule is None:
            schedule = ["simplicial" if layer % 2 == 0 else "knn_local" for layer in range(n_layers)]
        if len(schedule) != n_layers:
            raise ValueError("schedule must name one attention type per layer")
        self.knn_k = int(knn_k)
        self.schedule = list(schedule)
        self.blocks = nn.ModuleList([
            AdaLNBlock(d_model, n_heads, mlp_ratio=mlp_ratio, eps=eps, attn_type=t, simplicial_impl=simplicial_impl,
                       simplicial_precision=simplicial_precision, simplicial_message_mode=simplicial_message_mode,
                       simplicial_message_rank=simplicial_message_rank,
                       simplicial_content_logits=simplicial_content_logits, local_impl=local_impl,
                       use_adaln_conditioning=use_adaln_conditioning)
            for t in self.schedule])

    def _use_hip(self, x: torch.Tensor) -> bool:
        local = [b.attn for b in self.blocks if b.attn_type == "knn_local"]
        return x.device.type == "cuda" and any(a.impl != "torch" and a._hip_unavailable_reason(x) is None
                                               for a in local)

    def packable(self, x: torch.Tensor, terms: SimplicialTerms | None = None) -> bool:
        """True when every block would run its HIP kernels on x (with the simplicial terms of this call), which
        the packed forward requires."""
        if not self.pack_tokens or x.device.type != "cuda":
            return False
        t = terms or SimplicialTerms(None)
        for block in self.blocks:
            a = block.attn
            if a.impl == "torch":
                return False
            if block.attn_type == "knn_local":
                if a._hip_unavailable_reason(x) is not None:
                    return False
            elif a._triton_unavailable_reason(
                    x=x, factorized_bias=t.factorized_bias, angle_residual=t.angle_residual,
                    message_residual=t.message_residual,
                    message_basis=a.message_basis if t.message_residual is not None else None,
                    logit_bias_fn=t.logit_bias_fn, return_attn=False) is not None:
                return False
        return True

    def simplicial_terms(self, coords: torch.Tensor, pad_mask: torch.Tensor | None = None,
                         lattice: torch.Tensor | None = None, sigma: torch.Tensor | None = None
                         ) -> SimplicialTerms | None:
        """The geometry features and the simplicial blocks' bias / residual terms and attention mask, once per
        forward (TransformerTrunk.forward, transformer.py:1246-1296); None without a geometry adapter."""
        if self.geometry_adapter is None:
            return None
        geom = self.geometry_adapter(coords=coords, pad_mask=pad_mask, lattice=lattice)
        B, N = coords.shape[:2]
        if self.simplicial_geometry_bias is not None:
            fb, fn, ang, msg, mask = self.simplicial_geometry_bias.build_structured_bias_inputs(
                geom_features=geom, coords_len=N, pad_mask=pad_mask, seq_len=N, sigma=sigma)
            return SimplicialTerms(mask, fb, ang, msg, fn)
        from matterformer_amd.geometry_bias import build_simplicial_attention_mask

        mask = build_simplicial_attention_mask(coords_len=N, seq_len=N, batch_size=B, device=coords.device,
                                               pad_mask=pad_mask, geom_pair_mask=geom.pair_mask)
        return SimplicialTerms(mask)

    def forward(self, x: torch.Tensor, cond_emb: torch.Tensor | None, coords: torch.Tensor,
                pad_mask: torch.Tensor | None = None, *, lattice: torch.Tensor | None = None,
                sigma: torch.Tensor | None = None, packing: TokenPacking | None = None) -> torch.Tensor:
        """x (B, N, C) -> (B, N, C), padded rows zero.  With a geometry adapter (and a SimplicialGeometryBias)
        the simplicial blocks get the geometry attention mask and bias terms of (coords, lattice, sigma).
        ``packing`` (TokenPacking(pad_mask)) may be passed in, e.g. to capture the forward in a HIP graph;
        otherwise a GPU call with a pad_mask builds it."""
        if pad_mask is not None:
            pad_mask = pad_mask.bool()
        if packing is not None and (pad_mask is None or (packing.batch, packing.atoms) != tuple(pad_mask.shape)):
            raise ValueError("packing must be built from this call's pad_mask")
        explicit = packing is not None
        if pad_mask is not None and (explicit or self.packable(x)):
            # the packed forward: geometry features and simplicial terms straight on the compact layout
            # (each molecule's valid atoms first, width W), which is what the packed blocks read
            packing = packing if explicit else TokenPacking(pad_mask)
            cterms = self.simplicial_terms(packing.compact(coords), packing.compact_pad_mask, lattice, sigma)
            if self.packable(x, cterms):
                return self._forward_packed(x, cond_emb, coords, packing, cterms)
            if explicit:
                raise RuntimeError("the packed forward needs every block on its HIP kernels")
        terms = self.simplicial_terms(coords, pad_mask, lattice, sigma)
        mask = None
        if "knn_local" in self.schedule:
            mask = build_knn_mask(coords, self.knn_k, pad_mask, use_hip=self._use_hip(x))
        kwargs = terms.block_kwargs() if terms is not None else {}
        # transformer.py:1298-1316: padded atoms are zeroed before every block and in the output
        for block in self.blocks:
            if pad_mask is not None:
                x = x.masked_fill(pad_mask[..., None], 0.0)
            x = block(x, cond_emb, pad_mask, knn_mask=mask, **kwargs)
        if pad_mask is not None:
            x = x.masked_fill(pad_mask[..., None], 0.0)
        return x

    def _all_mods(self, cond_emb: torch.Tensor | None, batch: int) -> list[torch.Tensor]:
        """Every block's ada_ln(cond_emb) (B, 6C).  Without autograd: SiLU once and one GEMM over the blocks'
        concatenated ada_ln weights (the per-block GEMMs are a few microseconds of launch each)."""
        if cond_emb is None or cond_emb.ndim != 2 or cond_emb.shape[0] != batch:
            raise ValueError("cond_emb must have shape (B, C)")
        lins = [blk.ada_ln[-1] for blk in self.blocks]
        grad = torch.is_grad_enabled() and (cond_emb.requires_grad or any(l.weight.requires_grad for l in lins))
        if grad or cond_emb.device.type != "cuda":
            return [blk._mods(cond_emb, batch) for blk in self.blocks]
        w = torch.cat([lin.weight for lin in lins])
        b = torch.cat([lin.bias for lin in lins])
        out = F.linear(self.blocks[0].ada_ln[0](cond_emb), w, b)
        return list(out.split(lins[0].weight.shape[0], dim=1))

    def _forward_packed(self, x: torch.Tensor, cond_emb: torch.Tensor | None, coords: torch.Tensor,
                        packing: TokenPacking, terms: SimplicialTerms | None = None) -> torch.Tensor:
        """``terms``: the simplicial terms on the packing's compact layout (or None: key padding only)."""
        """The blocks on the valid rows; attention masks and kNN lists in the compact layout (each molecule's
        valid atoms first, width = its largest count).  With adaLN, one mf_adaln_rows pass joins each
        residual to the next LayerNorm + modulation, the last block's MLP residual to the next block's norm1."""
        B, W = packing.batch, packing.width
        cpad = packing.compact_pad_mask
        mask = None
        if "knn_local" in self.schedule:
            mask = build_knn_mask(packing.compact(coords.float()), self.knn_k, cpad, use_hip=True)
        if terms is None:
            terms = SimplicialTerms(coerce_attention_mask(None, key_padding_mask=cpad, batch_size=B, num_tokens=W,
                                                          device=x.device))
        xp = packing.pack(x)
        if not all(blk.use_adaln_conditioning for blk in self.blocks):
            for block in self.blocks:
                xp = block.forward_packed(xp, cond_emb, packing, knn_mask=mask, terms=terms)
            return packing.unpack(xp)
        C = xp.shape[-1]
        mods = self._all_mods(cond_emb, B)
        blocks = list(self.blocks)
        h = adaln_rows(packing, xp, shift=mods[0][:, :C], scale=mods[0][:, C:2 * C], eps=blocks[0].norm1.eps)
        for layer, blk in enumerate(blocks):
            m = mods[layer]
            a = blk._attention_packed(h, packing, mask, terms)
            xp, h = adaln_rows(packing, xp, a, gate=m[:, 2 * C:3 * C], shift=m[:, 3 * C:4 * C],
                               scale=m[:, 4 * C:5 * C], eps=blk.norm2.eps, inplace=layer > 0)
            y = blk.mlp(h)
            if layer + 1 < len(blocks):
                nxt = mods[layer + 1]
                xp, h = adaln_rows(packing, xp, y, gate=m[:, 5 * C:], shift=nxt[:, :C], scale=nxt[:, C:2 * C],
                                   eps=blocks[layer + 1].norm1.eps, inplace=True)
            else:
                xp = adaln_rows(packing, xp, y, gate=m[:, 5 * C:], inplace=True)
        return packing.unpack(xp)
