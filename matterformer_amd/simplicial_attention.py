"""2-simplicial attention module with HIP / torch backends.

Mirror of ``matterformer.models.simplicial_attention``
(src/matterformer/models/simplicial_attention.py): same public names,
constructor and forward signatures, dispatch rules and autograd contract.

  _TritonTwoSimplicialAttentionFunction  :347-637 (21 positional arguments;
      the kernels are looked up through the module globals
      ``triton_simplicial_attention_forward`` / ``_backward`` so callers and
      tests can swap them, as tests/test_simplicial_attention.py:755-756 does)
  SimplicialAttention                    :640-987
  TwoSimplicialAttention                 :990

``impl`` accepts "auto", "torch", "triton" (the reference name for the fused
backend, here the HIP kernel) and "hip" (same as "triton").  One deliberate
difference: on a GPU tensor, a missing HIP library is an error for "auto" too,
instead of a silent switch to the torch path.
"""

from __future__ import annotations

from typing import Callable

import torch
import torch.nn as nn

from matterformer_amd.hip_simplicial_attention import (
    TRITON_AVAILABLE,
    hip_unsupported_reason,
    normalize_simplicial_precision,
    triton_simplicial_attention_backward,
    triton_simplicial_attention_forward,
)
from matterformer_amd.simplicial_types import (
    SimplicialAttentionMask,
    SimplicialFactorizedBias,
    SimplicialLowRankAngleResidual,
    SimplicialLowRankMessageResidual,
    coerce_attention_mask,
    simplicial_attention_torch_from_projected,
)

__all__ = [
    "SimplicialAttention",
    "SimplicialAttentionMask",
    "SimplicialFactorizedBias",
    "SimplicialLowRankAngleResidual",
    "SimplicialLowRankMessageResidual",
    "TwoSimplicialAttention",
    "_TritonTwoSimplicialAttentionFunction",
    "simplicial_attention_torch_from_projected",
]

_coerce_attention_mask = coerce_attention_mask


def _canonicalize_simplicial_content_logits(mode: str) -> str:
    """Aliases of simplicial_attention.py:148-158."""
    mode = str(mode).lower().replace("-", "_")
    aliases = {
        "on": "on", "enabled": "on", "true": "on", "yes": "on",
        "off": "off", "disabled": "off", "false": "off", "no": "off",
        "learned": "learned", "gated": "learned", "learned_scale": "learned",
        "learnable": "learned", "learnable_scale": "learned",
    }
    if mode not in aliases:
        raise ValueError("simplicial_content_logits must be one of {'on', 'off', 'learned'}")
    return aliases[mode]


def _present(t: torch.Tensor) -> bool:
    return t.numel() > 0


class _TritonTwoSimplicialAttentionFunction(torch.autograd.Function):
    """Fused-kernel autograd wrapper; empty tensors mark absent optional inputs."""

    @staticmethod
    def forward(ctx, q, k1, v1, k2, v2, query_valid, pair_key_valid, pair_valid, u, v, w, gate,
                angle_left, angle_right, angle_gate, message_left, message_right, message_basis,
                precision_mode, chunk_size, debug_torch_backward):
        has_pv = _present(pair_valid)
        has_bias = _present(u)
        has_angle = _present(angle_left)
        has_message = _present(message_left)
        need_state = any(ctx.needs_input_grad)
        kwargs = dict(
            query_valid=query_valid,
            pair_key_valid=pair_key_valid,
            pair_valid=pair_valid if has_pv else None,
            u=u if has_bias else None,
            v_bias=v if has_bias else None,
            w=w if has_bias else None,
            gate=gate if has_bias else None,
            angle_left=angle_left if has_angle else None,
            angle_right=angle_right if has_angle else None,
            angle_gate=angle_gate if has_angle else None,
            message_left=message_left if has_message else None,
            message_right=message_right if has_message else None,
            message_basis=message_basis if has_message else None,
            precision=precision_mode,
        )
        if not need_state:
            kwargs["need_backward_state"] = False
        out, lse, out_f32 = triton_simplicial_attention_forward(q, k1, v1, k2, v2, **kwargs)
        ctx.precision_mode = str(precision_mode)
        ctx.chunk_size = int(chunk_size)
        ctx.debug_torch_backward = bool(debug_torch_backward)
        ctx.flags = (has_pv, has_bias, has_angle, has_message)
        if need_state:
            ctx.save_for_backward(q, k1, v1, k2, v2, query_valid, pair_key_valid, pair_valid, u, v, w, gate,
                                  angle_left, angle_right, angle_gate, message_left, message_right,
                                  message_basis, out_f32, lse)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        (q, k1, v1, k2, v2, query_valid, pair_key_valid, pair_valid, u, v, w, gate, angle_left, angle_right,
         angle_gate, message_left, message_right, message_basis, out, lse) = ctx.saved_tensors
        has_pv, has_bias, has_angle, has_message = ctx.flags
        if ctx.debug_torch_backward:
            grads = _debug_torch_backward(ctx, grad_out, q, k1, v1, k2, v2, query_valid, pair_key_valid,
                                          pair_valid, u, v, w, gate, angle_left, angle_right, angle_gate,
                                          message_left, message_right, message_basis)
            return (*grads[:5], None, None, None, *grads[5:], None, None, None)
        nig = ctx.needs_input_grad
        result = triton_simplicial_attention_backward(
            grad_out, q, k1, v1, k2, v2, out, lse,
            query_valid=query_valid,
            pair_key_valid=pair_key_valid,
            pair_valid=pair_valid if has_pv else None,
            u=u if has_bias else None,
            v_bias=v if has_bias else None,
            w=w if has_bias else None,
            gate=gate if has_bias else None,
            angle_left=angle_left if has_angle else None,
            angle_right=angle_right if has_angle else None,
            angle_gate=angle_gate if has_angle else None,
            message_left=message_left if has_message else None,
            message_right=message_right if has_message else None,
            message_basis=message_basis if has_message else None,
            precision=ctx.precision_mode,
            need_du=bool(has_bias and nig[8]),
            need_dv_bias=bool(has_bias and nig[9]),
            need_dw=bool(has_bias and nig[10]),
            need_dgate=bool(has_bias and nig[11]),
            need_dangle_left=bool(has_angle and nig[12]),
            need_dangle_right=bool(has_angle and nig[13]),
            need_dangle_gate=bool(has_angle and nig[14]),
            need_dmessage_left=bool(has_message and nig[15]),
            need_dmessage_right=bool(has_message and nig[16]),
            need_dmessage_basis=bool(has_message and nig[17]),
        )
        return (*result[:5], None, None, None, *result[5:], None, None, None)


def _debug_torch_backward(ctx, grad_out, q, k1, v1, k2, v2, query_valid, pair_key_valid, pair_valid, u, v, w,
                          gate, angle_left, angle_right, angle_gate, message_left, message_right, message_basis):
    """Recompute with the fp32-core torch path and autograd (simplicial_attention.py:454-552)."""
    has_pv, has_bias, has_angle, has_message = ctx.flags
    core = [t.detach().requires_grad_(True) for t in (q, k1, v1, k2, v2)]
    groups = []
    for present, tensors in ((has_bias, (u, v, w, gate)), (has_angle, (angle_left, angle_right, angle_gate)),
                             (has_message, (message_left, message_right, message_basis))):
        groups.append([t.detach().requires_grad_(True) for t in tensors] if present else None)
    with torch.enable_grad():
        fb = SimplicialFactorizedBias(*groups[0]) if groups[0] else None
        ar = SimplicialLowRankAngleResidual(*groups[1]) if groups[1] else None
        mr = SimplicialLowRankMessageResidual(left=groups[2][0], right=groups[2][1]) if groups[2] else None
        mask = SimplicialAttentionMask(query_valid=query_valid, pair_key_valid=pair_key_valid,
                                       pair_valid=pair_valid if has_pv else None)
        ref = simplicial_attention_torch_from_projected(
            *core, attention_mask=mask, factorized_bias=fb, angle_residual=ar, message_residual=mr,
            message_basis=groups[2][2] if groups[2] else None, chunk_size=ctx.chunk_size, fp32_core=True,
        )
        inputs = core + [t for grp in groups if grp for t in grp]
        grads = list(torch.autograd.grad(ref, inputs, grad_out, allow_unused=True))
    full = grads[:5]
    cursor = 5
    for grp, size in zip(groups, (4, 3, 3)):
        if grp:
            full.extend(grads[cursor:cursor + size])
            cursor += size
        else:
            full.extend([None] * size)
    return full


class SimplicialAttention(nn.Module):
    """Dense non-causal 2-simplicial attention with explicit torch / HIP backends."""

    def __init__(
        self,
        dim: int,
        num_heads: int,
        *,
        head_dim: int | None = None,
        dropout: float = 0.0,
        bias: bool = True,
        chunk_size: int = 128,
        out_proj: bool = True,
        impl: str = "auto",
        precision: str = "bf16_tc",
        message_mode: str = "none",
        message_rank: int = 16,
        content_logits: str = "on",
        debug_torch_backward: bool = False,
    ) -> None:
        super().__init__()
        if head_dim is None:
            if dim % num_heads != 0:
                raise ValueError(f"dim ({dim}) must be divisible by num_heads ({num_heads}) when head_dim is None.")
            head_dim = dim // num_heads
        if head_dim <= 0:
            raise ValueError("head_dim must be positive")
        if chunk_size <= 0:
            raise ValueError("chunk_size must be positive")
        impl = impl.lower()
        if impl == "hip":
            impl = "triton"
        if impl not in {"auto", "torch", "triton"}:
            raise ValueError(f"Unsupported simplicial_impl: {impl}")
        message_mode = message_mode.lower()
        if message_mode not in {"none", "low_rank"}:
            raise ValueError(f"Unsupported simplicial_message_mode: {message_mode}")
        message_rank = int(message_rank)
        if message_mode == "low_rank" and message_rank <= 0:
            raise ValueError("simplicial_message_rank must be positive when message_mode='low_rank'")

        self.dim = int(dim)
        self.num_heads = int(num_heads)
        self.head_dim = int(head_dim)
        self.inner_dim = self.num_heads * self.head_dim
        self.dropout = float(dropout)
        self.chunk_size = int(chunk_size)
        self.impl = impl
        self.precision = normalize_simplicial_precision(precision)
        self.message_mode = message_mode
        self.message_rank = message_rank
        self.content_logits = _canonicalize_simplicial_content_logits(content_logits)
        self.debug_torch_backward = bool(debug_torch_backward)
        self.scale = self.head_dim ** -0.5
        self._last_impl_used = "torch"

        self.in_proj = nn.Linear(self.dim, 5 * self.inner_dim, bias=bias)
        self.out_proj = nn.Linear(self.inner_dim, self.dim, bias=bias) if out_proj else nn.Identity()
        if self.message_mode == "low_rank":
            self.message_basis = nn.Parameter(torch.empty(self.num_heads, self.message_rank, self.head_dim))
            nn.init.normal_(self.message_basis, mean=0.0, std=self.head_dim ** -0.5)
        else:
            self.message_basis = None
        if self.content_logits == "learned":
            self.content_logit_log_scale = nn.Parameter(torch.zeros((1, self.num_heads, 1, 1), dtype=torch.float32))
        else:
            self.content_logit_log_scale = None

    @staticmethod
    def _split_heads(x: torch.Tensor, num_heads: int, head_dim: int) -> torch.Tensor:
        B, T, _ = x.shape
        return x.view(B, T, num_heads, head_dim).transpose(1, 2)

    @staticmethod
    def _merge_heads(x: torch.Tensor) -> torch.Tensor:
        B, H, T, D = x.shape
        return x.transpose(1, 2).contiguous().view(B, T, H * D)

    def _project_inputs(self, x: torch.Tensor):
        parts = self.in_proj(x).chunk(5, dim=-1)
        heads = [self._split_heads(p, self.num_heads, self.head_dim) for p in parts]
        heads[0] = heads[0] * self.scale
        return tuple(heads)

    def _content_query(self, q: torch.Tensor) -> torch.Tensor:
        if self.content_logits == "on":
            return q
        if self.content_logits == "off":
            return torch.zeros_like(q)
        return q * self.content_logit_log_scale.to(device=q.device, dtype=q.dtype).exp()

    def _triton_unavailable_reason(
        self,
        *,
        x: torch.Tensor,
        factorized_bias: SimplicialFactorizedBias | None,
        angle_residual: SimplicialLowRankAngleResidual | None,
        message_residual: SimplicialLowRankMessageResidual | None,
        message_basis: torch.Tensor | None,
        logit_bias_fn: Callable | None,
        return_attn: bool,
    ) -> str | None:
        """None when the fused HIP kernel can serve the call (simplicial_attention.py:735-782)."""
        if not TRITON_AVAILABLE:
            return "the HIP library is not built"
        if x.device.type != "cuda":
            return "the HIP backend requires GPU tensors"
        if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            return f"the HIP backend only supports float16/bfloat16/float32 inputs, got {x.dtype}"
        if self.training and self.dropout > 0.0:
            return "the HIP backend does not support attention dropout in training mode"
        if return_attn:
            return "the HIP backend does not support return_attn=True"
        if logit_bias_fn is not None:
            return "the HIP backend does not support arbitrary Python logit_bias_fn callbacks"
        if self.head_dim > 128:
            return f"the HIP backend only supports head_dim <= 128, got {self.head_dim}"
        if factorized_bias is not None:
            for name, tensor in (("u", factorized_bias.u), ("v", factorized_bias.v), ("w", factorized_bias.w),
                                 ("gate", factorized_bias.gate)):
                if tensor.device != x.device:
                    return f"factorized bias tensor {name} must be on the same GPU device as the attention input"
        if angle_residual is not None:
            if any(t.device != x.device for t in (angle_residual.left, angle_residual.right, angle_residual.gate)):
                return "angle residual tensors must be on the same GPU device as the attention input"
            if angle_residual.rank > 64:
                return f"the HIP backend only supports low-rank angle residual rank <= 64, got {angle_residual.rank}"
        if message_residual is not None:
            if message_basis is None:
                return "message residual tensors require a message_basis"
            if message_residual.left.device != x.device or message_residual.right.device != x.device:
                return "message residual tensors must be on the same GPU device as the attention input"
            if message_basis.device != x.device:
                return "message basis tensor must be on the same GPU device as the attention input"
            expected = (self.num_heads, message_residual.rank, self.head_dim)
            if tuple(message_basis.shape) != expected:
                return f"message basis tensor must have shape {expected}, got {tuple(message_basis.shape)}"
            if message_residual.rank > 64:
                return f"the HIP backend only supports low-rank message residual rank <= 64, got {message_residual.rank}"
        elif message_basis is not None:
            return "message_basis must be None when message_residual is None"
        return hip_unsupported_reason(x.shape[0], self.num_heads, x.shape[1], self.head_dim,
                                      self._triton_compute_dtype())

    def _triton_compute_dtype(self) -> torch.dtype:
        return torch.bfloat16 if self.precision == "bf16_tc" else torch.float32

    def _forward_triton(self, q, k1, v1, k2, v2, *, attention_mask, factorized_bias, angle_residual,
                        message_residual, message_basis):
        mask = coerce_attention_mask(attention_mask, key_padding_mask=None, batch_size=q.shape[0],
                                     num_tokens=q.shape[2], device=q.device)
        cdt = self._triton_compute_dtype()
        q, k1, v1, k2, v2 = (t.to(dtype=cdt) for t in (q, k1, v1, k2, v2))
        empty = q.new_empty(0)
        empty_bool = torch.empty(0, device=q.device, dtype=torch.bool)
        if factorized_bias is None:
            u = vb = w = gate = empty
        else:
            factorized_bias.validate(batch_size=q.shape[0], num_heads=q.shape[1], num_tokens=q.shape[2])
            u, vb, w, gate = factorized_bias.u, factorized_bias.v, factorized_bias.w, factorized_bias.gate
        if angle_residual is None:
            al = ar_ = ag = empty
        else:
            angle_residual.validate(batch_size=q.shape[0], num_heads=q.shape[1], num_tokens=q.shape[2])
            al, ar_, ag = (t.float() for t in (angle_residual.left, angle_residual.right, angle_residual.gate))
        if message_residual is None:
            ml = mr = mb = empty
        else:
            if message_basis is None:
                raise RuntimeError("message_residual requires message_basis")
            message_residual.validate(batch_size=q.shape[0], num_heads=q.shape[1], num_tokens=q.shape[2])
            ml, mr = message_residual.left.float(), message_residual.right.float()
            mb = message_basis.to(device=q.device, dtype=torch.float32)
        pv = mask.pair_valid.contiguous() if mask.pair_valid is not None else empty_bool
        # q, k1, v1, k2, v2 stay the head views of the in_proj output (the reference copies them with
        # .contiguous() here): the launcher reads them in place through their strides when its kernel
        # can, and makes the copies itself otherwise
        return _TritonTwoSimplicialAttentionFunction.apply(
            q, k1, v1, k2, v2,
            mask.query_valid.contiguous(), mask.pair_key_valid.contiguous(), pv,
            u.contiguous(), vb.contiguous(), w.contiguous(), gate.contiguous(),
            al.contiguous(), ar_.contiguous(), ag.contiguous(),
            ml.contiguous(), mr.contiguous(), mb.contiguous(),
            self.precision, self.chunk_size, self.debug_torch_backward,
        )

    def forward(
        self,
        x: torch.Tensor,
        *,
        key_padding_mask: torch.Tensor | None = None,
        attention_mask: SimplicialAttentionMask | None = None,
        factorized_bias: SimplicialFactorizedBias | None = None,
        angle_residual: SimplicialLowRankAngleResidual | None = None,
        message_residual: SimplicialLowRankMessageResidual | None = None,
        logit_bias_fn: Callable[[int, int, torch.dtype, torch.device], torch.Tensor] | None = None,
        return_attn: bool = False,
    ):
        if x.ndim != 3:
            raise ValueError(f"x must have shape (B, T, C), got {tuple(x.shape)}")
        B, T, _ = x.shape
        attention_mask = coerce_attention_mask(attention_mask, key_padding_mask=key_padding_mask, batch_size=B,
                                               num_tokens=T, device=x.device)
        if factorized_bias is not None:
            factorized_bias.validate(batch_size=B, num_heads=self.num_heads, num_tokens=T)
        if angle_residual is not None:
            angle_residual.validate(batch_size=B, num_heads=self.num_heads, num_tokens=T)
        if message_residual is not None:
            if self.message_basis is None:
                raise ValueError("message_residual requires simplicial_message_mode='low_rank'")
            message_residual.validate(batch_size=B, num_heads=self.num_heads, num_tokens=T)
            if message_residual.rank != self.message_rank:
                raise ValueError(
                    f"message_residual rank {message_residual.rank} does not match attention message_rank "
                    f"{self.message_rank}"
                )
        message_basis = self.message_basis if message_residual is not None else None

        # The dispatch decision depends only on x and the module, so it is taken
        # before the projection: an explicit impl="triton" call with an
        # unsupported input dtype then fails with the backend's own message
        # (the behaviour tests/test_simplicial_attention.py:819-824 expects)
        # rather than inside in_proj.
        reason = self._triton_unavailable_reason(
            x=x, factorized_bias=factorized_bias, angle_residual=angle_residual, message_residual=message_residual,
            message_basis=message_basis, logit_bias_fn=logit_bias_fn, return_attn=return_attn,
        )
        if x.device.type == "cuda" and not TRITON_AVAILABLE and self.impl != "torch":
            raise RuntimeError(f"HIP simplicial attention library missing on a GPU host: {reason}")
        if self.impl == "auto":
            impl_used = "triton" if reason is None else "torch"
        elif self.impl == "triton":
            if reason is not None:
                raise RuntimeError(f"HIP simplicial attention is unavailable: {reason}")
            impl_used = "triton"
        else:
            impl_used = "torch"
        self._last_impl_used = impl_used

        q, k1, v1, k2, v2 = self._project_inputs(x)
        q_content = self._content_query(q)

        if impl_used == "triton":
            out = self._forward_triton(
                q_content, k1, v1, k2, v2, attention_mask=attention_mask, factorized_bias=factorized_bias,
                angle_residual=angle_residual, message_residual=message_residual, message_basis=message_basis,
            )
            return self.out_proj(self._merge_heads(out.to(x.dtype)))

        out = simplicial_attention_torch_from_projected(
            q_content, k1, v1, k2, v2, attention_mask=attention_mask, factorized_bias=factorized_bias,
            angle_residual=angle_residual, message_residual=message_residual, message_basis=message_basis,
            logit_bias_fn=logit_bias_fn, dropout_p=self.dropout, training=self.training,
            chunk_size=self.chunk_size, return_attn=return_attn,
        )
        if return_attn:
            heads, attn = out
            return self.out_proj(self._merge_heads(heads)), attn
        return self.out_proj(self._merge_heads(out))


TwoSimplicialAttention = SimplicialAttention
