"""Structured inputs of 2-simplicial attention and the reference torch path.

These mirror the reference's public types and its ``impl="torch"`` backend
(``src/matterformer/models/simplicial_attention.py``):

  SimplicialFactorizedBias          :18-47
  SimplicialLowRankAngleResidual    :50-81
  SimplicialLowRankMessageResidual  :84-104
  SimplicialAttentionMask           :107-145
  simplicial_attention_torch_from_projected  :206-344

The torch path is the reference's chunked algorithm (it materialises logits
for a block of queries in fp32, masks invalid pairs with ``finfo.min`` and takes
one softmax over all (j,k) pairs); its steps must match the reference to
reproduce its bf16 rounding, so they follow it step for step.  It is what
``SimplicialAttention(impl="torch")`` runs and what ``impl="auto"`` uses off
the GPU or for features the HIP kernel does not cover (a Python
``logit_bias_fn``, ``return_attn``, training-mode dropout), exactly as the
reference dispatches.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

import torch
import torch.nn.functional as F


@dataclass(frozen=True)
class SimplicialFactorizedBias:
    """gate_i * (u_ij + v_ik + w_jk); u, v, w: (B,H,T,T), gate: (B,H,T)."""

    u: torch.Tensor
    v: torch.Tensor
    w: torch.Tensor
    gate: torch.Tensor

    def validate(self, *, batch_size: int, num_heads: int, num_tokens: int) -> None:
        pair_shape = (batch_size, num_heads, num_tokens, num_tokens)
        for name in ("u", "v", "w"):
            got = tuple(getattr(self, name).shape)
            if got != pair_shape:
                raise ValueError(f"{name} must have shape {pair_shape}, got {got}")
        gate_shape = (batch_size, num_heads, num_tokens)
        if tuple(self.gate.shape) != gate_shape:
            raise ValueError(f"gate must have shape {gate_shape}, got {tuple(self.gate.shape)}")

    def chunk(self, start: int, end: int, *, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
        """Bias for queries [start, end): (B,H,end-start,T,T), summed in fp32."""
        u = self.u[:, :, start:end].float()[..., :, None]
        v = self.v[:, :, start:end].float()[..., None, :]
        w = self.w.float()[:, :, None]
        gate = self.gate[:, :, start:end].float()[..., None, None]
        return (gate * (u + v + w)).to(device=device, dtype=dtype)


@dataclass(frozen=True)
class SimplicialLowRankAngleResidual:
    """gate_i * R^-1/2 * sum_r left_ijr right_ikr; left/right: (B,H,T,T,R), gate: (B,H,T)."""

    left: torch.Tensor
    right: torch.Tensor
    gate: torch.Tensor

    @property
    def rank(self) -> int:
        return int(self.left.shape[-1])

    def validate(self, *, batch_size: int, num_heads: int, num_tokens: int) -> None:
        _validate_low_rank(self.left, self.right, batch_size, num_heads, num_tokens, "angle")
        gate_shape = (batch_size, num_heads, num_tokens)
        if tuple(self.gate.shape) != gate_shape:
            raise ValueError(f"gate must have shape {gate_shape}, got {tuple(self.gate.shape)}")

    def chunk(self, start: int, end: int, *, dtype: torch.dtype, device: torch.device) -> torch.Tensor:
        left = self.left[:, :, start:end].float()
        right = self.right[:, :, start:end].float()
        res = torch.einsum("bhqjr,bhqkr->bhqjk", left, right) * (self.rank ** -0.5)
        gate = self.gate[:, :, start:end].float()[..., None, None]
        return (gate * res).to(device=device, dtype=dtype)


@dataclass(frozen=True)
class SimplicialLowRankMessageResidual:
    """Message term c_ir = R^-1/2 sum_jk P_ijk left_ijr right_ikr; out += c @ basis."""

    left: torch.Tensor
    right: torch.Tensor

    @property
    def rank(self) -> int:
        return int(self.left.shape[-1])

    def validate(self, *, batch_size: int, num_heads: int, num_tokens: int) -> None:
        _validate_low_rank(self.left, self.right, batch_size, num_heads, num_tokens, "message")


def _validate_low_rank(left, right, batch_size, num_heads, num_tokens, kind: str) -> None:
    if left.ndim != 5:
        raise ValueError(f"left must have shape (B, H, T, T, R), got {tuple(left.shape)}")
    prefix = (batch_size, num_heads, num_tokens, num_tokens)
    if tuple(left.shape[:4]) != prefix:
        raise ValueError(f"left must have shape {prefix + (left.shape[-1],)}, got {tuple(left.shape)}")
    if right.shape != left.shape:
        raise ValueError(f"right must have shape {tuple(left.shape)}, got {tuple(right.shape)}")
    if int(left.shape[-1]) <= 0:
        raise ValueError(f"low-rank {kind} residual rank must be positive")


@dataclass(frozen=True)
class SimplicialAttentionMask:
    """query_valid (B,T), pair_key_valid (B,T), optional pair_valid (B,T,T); True = valid."""

    query_valid: torch.Tensor
    pair_key_valid: torch.Tensor
    pair_valid: torch.Tensor | None = None

    def validate(self, *, batch_size: int, num_tokens: int) -> None:
        shape = (batch_size, num_tokens)
        if tuple(self.query_valid.shape) != shape:
            raise ValueError(f"query_valid must have shape {shape}, got {tuple(self.query_valid.shape)}")
        if tuple(self.pair_key_valid.shape) != shape:
            raise ValueError(f"pair_key_valid must have shape {shape}, got {tuple(self.pair_key_valid.shape)}")
        if self.pair_valid is not None and tuple(self.pair_valid.shape) != (batch_size, num_tokens, num_tokens):
            raise ValueError(
                f"pair_valid must have shape {(batch_size, num_tokens, num_tokens)}, got {tuple(self.pair_valid.shape)}"
            )

    @classmethod
    def from_key_padding_mask(
        cls,
        key_padding_mask: torch.Tensor | None,
        *,
        batch_size: int,
        num_tokens: int,
        device: torch.device,
    ) -> "SimplicialAttentionMask":
        """key_padding_mask uses True = padding (nn.MultiheadAttention convention)."""
        if key_padding_mask is None:
            valid = torch.ones(batch_size, num_tokens, device=device, dtype=torch.bool)
        else:
            if tuple(key_padding_mask.shape) != (batch_size, num_tokens):
                raise ValueError(
                    f"key_padding_mask must have shape {(batch_size, num_tokens)}, got {tuple(key_padding_mask.shape)}"
                )
            valid = ~key_padding_mask.to(device=device).bool()
        return cls(query_valid=valid, pair_key_valid=valid)

    def pair_mask(self) -> torch.Tensor:
        keys = self.pair_key_valid.bool()
        mask = keys[:, :, None] & keys[:, None, :]
        if self.pair_valid is not None:
            mask = mask & self.pair_valid.bool()
        return mask


def coerce_attention_mask(
    attention_mask: SimplicialAttentionMask | None,
    *,
    key_padding_mask: torch.Tensor | None,
    batch_size: int,
    num_tokens: int,
    device: torch.device,
) -> SimplicialAttentionMask:
    """Build/validate the mask and move it to ``device`` as bool (simplicial_attention.py:183-203)."""
    if attention_mask is None:
        attention_mask = SimplicialAttentionMask.from_key_padding_mask(
            key_padding_mask, batch_size=batch_size, num_tokens=num_tokens, device=device
        )
    attention_mask.validate(batch_size=batch_size, num_tokens=num_tokens)
    pv = attention_mask.pair_valid
    return SimplicialAttentionMask(
        query_valid=attention_mask.query_valid.to(device=device).bool(),
        pair_key_valid=attention_mask.pair_key_valid.to(device=device).bool(),
        pair_valid=None if pv is None else pv.to(device=device).bool(),
    )


def _as_fp32(x):
    if x is None:
        return None
    if isinstance(x, SimplicialFactorizedBias):
        return SimplicialFactorizedBias(u=x.u.float(), v=x.v.float(), w=x.w.float(), gate=x.gate.float())
    if isinstance(x, SimplicialLowRankAngleResidual):
        return SimplicialLowRankAngleResidual(left=x.left.float(), right=x.right.float(), gate=x.gate.float())
    if isinstance(x, SimplicialLowRankMessageResidual):
        return SimplicialLowRankMessageResidual(left=x.left.float(), right=x.right.float())
    return x.float()


def simplicial_attention_torch_from_projected(
    q: torch.Tensor,
    k1: torch.Tensor,
    v1: torch.Tensor,
    k2: torch.Tensor,
    v2: torch.Tensor,
    *,
    key_padding_mask: torch.Tensor | None = None,
    attention_mask: SimplicialAttentionMask | None = None,
    factorized_bias: SimplicialFactorizedBias | None = None,
    angle_residual: SimplicialLowRankAngleResidual | None = None,
    message_residual: SimplicialLowRankMessageResidual | None = None,
    message_basis: torch.Tensor | None = None,
    logit_bias_fn: Callable[[int, int, torch.dtype, torch.device], torch.Tensor] | None = None,
    dropout_p: float = 0.0,
    training: bool = False,
    chunk_size: int = 128,
    return_attn: bool = False,
    fp32_core: bool = False,
) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor]:
    """Reference torch path on ``(B,H,T,D)`` projections (simplicial_attention.py:206-344)."""
    B, H, T, D = q.shape
    if factorized_bias is not None:
        factorized_bias.validate(batch_size=B, num_heads=H, num_tokens=T)
    if angle_residual is not None:
        angle_residual.validate(batch_size=B, num_heads=H, num_tokens=T)
    if message_residual is not None:
        message_residual.validate(batch_size=B, num_heads=H, num_tokens=T)
        if message_basis is None:
            raise ValueError("message_basis must be provided when message_residual is provided")
        if tuple(message_basis.shape) != (H, message_residual.rank, D):
            raise ValueError(
                f"message_basis must have shape {(H, message_residual.rank, D)}, got {tuple(message_basis.shape)}"
            )
    elif message_basis is not None:
        raise ValueError("message_basis must be None when message_residual is None")

    mask = coerce_attention_mask(attention_mask, key_padding_mask=key_padding_mask, batch_size=B,
                                 num_tokens=T, device=q.device)
    flat_mask = mask.pair_mask()[:, None, None].flatten(-2)  # (B,1,1,T*T)
    query_valid = mask.query_valid

    upcast = fp32_core and q.dtype in (torch.float16, torch.bfloat16)
    if upcast:
        q, k1, v1w, k2, v2 = (t.float() for t in (q, k1, v1, k2, v2))
        factorized_bias, angle_residual, message_residual, message_basis = (
            _as_fp32(factorized_bias), _as_fp32(angle_residual), _as_fp32(message_residual), _as_fp32(message_basis)
        )
        out_dtype = torch.float32
    else:
        v1w = v1
        out_dtype = v1.dtype

    out = torch.empty((B, H, T, D), device=q.device, dtype=out_dtype)
    attn_parts: list[torch.Tensor] = []
    for start in range(0, T, chunk_size):
        end = min(T, start + chunk_size)
        qk2 = q[:, :, start:end, None, :] * k2[:, :, None, :, :]
        logits = torch.matmul(k1[:, :, None, :, :], qk2.transpose(-1, -2)).float()
        if factorized_bias is not None:
            logits = logits + factorized_bias.chunk(start, end, dtype=logits.dtype, device=logits.device)
        if angle_residual is not None:
            logits = logits + angle_residual.chunk(start, end, dtype=logits.dtype, device=logits.device)
        if logit_bias_fn is not None:
            logits = logits + logit_bias_fn(start, end, logits.dtype, logits.device)
        flat = logits.flatten(-2).masked_fill(~flat_mask, torch.finfo(logits.dtype).min)
        attn = torch.softmax(flat, dim=-1)
        attn = torch.where(flat_mask, attn, torch.zeros_like(attn)).view_as(logits)
        if dropout_p > 0.0:
            attn = F.dropout(attn, p=dropout_p, training=training)
        if return_attn:
            attn_parts.append(attn.detach())
        tmp = torch.matmul(attn.to(v1w.dtype).transpose(-2, -1), v1w[:, :, None, :, :])
        part = (tmp * v2[:, :, None, :, :]).sum(dim=-2)
        if message_residual is not None and message_basis is not None:
            coeff = torch.einsum(
                "bhqjk,bhqjr,bhqkr->bhqr",
                attn.float(),
                message_residual.left[:, :, start:end].float(),
                message_residual.right[:, :, start:end].float(),
            ) * (message_residual.rank ** -0.5)
            part = part + torch.einsum("bhqr,hrd->bhqd", coeff, message_basis.float()).to(part.dtype)
        part = part * query_valid[:, start:end].to(part.dtype)[:, None, :, None]
        out[:, :, start:end] = part
    if return_attn:
        return out.to(v1.dtype), torch.cat(attn_parts, dim=2)
    return out.to(v1.dtype)
