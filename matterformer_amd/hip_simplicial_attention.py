"""HIP backend of 2-simplicial attention: host side of ``mf_simplicial_fwd``.

Drop-in for ``matterformer.models.triton_simplicial_attention``
(src/matterformer/models/triton_simplicial_attention.py).  Same names, argument
meaning and return contract:

  TRITON_AVAILABLE                  :12   -> the HIP library is loadable
  SUPPORTED_SIMPLICIAL_PRECISIONS   :13
  normalize_simplicial_precision    :19-25
  triton_block_d_for_head_dim       :28-39
  triton_simplicial_attention_forward   :790-926 -> hip_simplicial_attention_forward
  triton_simplicial_attention_backward  :929-1204 -> hip_simplicial_attention_backward

The forward is one launch of the hand-written gfx950 kernels through the C ABI
(include/mf_capi.h), factorized bias, low-rank angle and message terms
included; a missing library, a CPU tensor or an unsupported shape raises
RuntimeError.  The backward is one launch of the deterministic HIP backward
kernel, except for calls with low-rank angle / message terms (and shapes
beyond that kernel's LDS capacity), whose gradients come from the reference's
own fp32-core recompute on the same device; ``last_backward_impl`` says which
ran.
"""

from __future__ import annotations

import ctypes

import torch

from matterformer_amd import _native
from matterformer_amd.simplicial_types import (
    SimplicialAttentionMask,
    SimplicialFactorizedBias,
    SimplicialLowRankAngleResidual,
    SimplicialLowRankMessageResidual,
    simplicial_attention_torch_from_projected,
)

HIP_AVAILABLE = _native.is_loaded()
# The reference's flag name; True means the fused (here: HIP) backend is usable.
TRITON_AVAILABLE = HIP_AVAILABLE
SUPPORTED_SIMPLICIAL_PRECISIONS = ("bf16_tc", "tf32", "ieee_fp32")


def normalize_simplicial_precision(precision: str) -> str:
    normalized = str(precision).lower()
    if normalized not in SUPPORTED_SIMPLICIAL_PRECISIONS:
        raise ValueError(
            f"Unsupported simplicial_precision: {precision}. Expected one of {SUPPORTED_SIMPLICIAL_PRECISIONS}."
        )
    return normalized


def triton_block_d_for_head_dim(head_dim: int) -> int:
    """Padded head dim used by the reference kernel (kept for API compatibility)."""
    if head_dim <= 0:
        raise ValueError("head_dim must be positive")
    for block in (16, 32, 64, 128):
        if head_dim <= block:
            return block
    raise ValueError(f"Triton simplicial attention only supports head_dim <= 128, got {head_dim}")


def hip_block_d_for_head_dim(head_dim: int) -> int:
    """Padded head dim of the HIP kernel's MFMA tiles (32, 64 or 128)."""
    return max(32, triton_block_d_for_head_dim(head_dim))


def hip_unsupported_reason(batch: int, heads: int, tokens: int, head_dim: int, dtype: torch.dtype) -> str | None:
    """None if mf_simplicial_fwd serves this shape, else the library's reason."""
    if not HIP_AVAILABLE:
        return f"the HIP library is unavailable: {_native.load_error()}"
    if dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return f"the HIP backend only supports float16/bfloat16/float32 inputs, got {dtype}"
    lib = _native.lib()
    status = lib.mf_simplicial_fwd_supported(batch, heads, tokens, head_dim, _native.dtype_code(dtype))
    if status != _native.MF_OK:
        return _native.last_error()
    return None


def _compute_dtype(dtype: torch.dtype, precision: str) -> torch.dtype:
    # bf16_tc keeps 16-bit operands on 16-bit MFMA; tf32/ieee_fp32 upcast 16-bit
    # operands to fp32 (the reference's USE_FP32_INPUT, triton...py:62-68).
    # fp32 operands always run the fp32 MFMA path.
    if precision == "bf16_tc" and dtype in (torch.bfloat16, torch.float16):
        return dtype
    return torch.float32


class _Extras:
    """Device tensors of the optional terms, laid out as mf_simplicial_fwd reads them."""

    def __init__(self):
        self.bias = None      # (u, v, w, gate) [B*H,N,N] x3, [B*H,N]; one dtype
        self.angle = None     # (left, right, gate) fp32
        self.message = None   # (left, right, basis) fp32

    @property
    def present(self) -> bool:
        return self.bias is not None or self.angle is not None or self.message is not None

    def fields(self) -> dict:
        f = {}
        if self.bias is not None:
            u, v, w, g = self.bias
            f.update(bias_u=u.data_ptr(), bias_v=v.data_ptr(), bias_w=w.data_ptr(), bias_gate=g.data_ptr(),
                     bias_dtype=_native.dtype_code(u.dtype))
        if self.angle is not None:
            left, right, g = self.angle
            f.update(angle_left=left.data_ptr(), angle_right=right.data_ptr(), angle_gate=g.data_ptr(),
                     angle_rank=int(left.shape[-1]))
        if self.message is not None:
            left, right, basis = self.message
            f.update(message_left=left.data_ptr(), message_right=right.data_ptr(),
                     message_basis=basis.data_ptr(), message_rank=int(left.shape[-1]))
        return f


def _on_device(name: str, t: torch.Tensor, device: torch.device, shape: tuple) -> torch.Tensor:
    if t.device != device:
        raise RuntimeError(f"{name} must be on {device}, got {t.device}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    return t


def _prepare_extras(q, B, H, N, D, u, v_bias, w, gate, angle_left, angle_right, angle_gate,
                    message_left, message_right, message_basis) -> _Extras:
    """Presence rules and checks of the reference launcher (triton_simplicial_attention.py:827-871):
    a group is used only when all its tensors are given; the bias keeps its dtype (fp32 if it is
    none of fp16/bf16/fp32), the rank factors are read as fp32."""
    ext = _Extras()
    dev = q.device
    if u is not None and v_bias is not None and w is not None and gate is not None:
        tensors = [_on_device(n, t, dev, s) for n, t, s in (
            ("u", u, (B, H, N, N)), ("v_bias", v_bias, (B, H, N, N)), ("w", w, (B, H, N, N)),
            ("gate", gate, (B, H, N)))]
        dt = tensors[0].dtype
        if dt not in (torch.float32, torch.float16, torch.bfloat16) or any(t.dtype != dt for t in tensors):
            dt = torch.float32
        ext.bias = tuple(t.to(dt).contiguous() for t in tensors)
    if angle_left is not None and angle_right is not None and angle_gate is not None:
        if angle_left.shape != angle_right.shape:
            raise ValueError(
                f"angle_left and angle_right must have the same shape, got {angle_left.shape} and {angle_right.shape}")
        rank = int(angle_left.shape[-1])
        if rank > 64:
            raise ValueError(f"the HIP kernel only supports low-rank features <= 64, got {rank}")
        ext.angle = tuple(_on_device(n, t, dev, s).float().contiguous() for n, t, s in (
            ("angle_left", angle_left, (B, H, N, N, rank)), ("angle_right", angle_right, (B, H, N, N, rank)),
            ("angle_gate", angle_gate, (B, H, N))))
    if message_left is not None and message_right is not None and message_basis is not None:
        if message_left.shape != message_right.shape:
            raise ValueError(
                f"message_left and message_right must have the same shape, got {message_left.shape} and "
                f"{message_right.shape}")
        rank = int(message_left.shape[-1])
        if tuple(message_basis.shape) != (H, rank, D):
            raise ValueError(f"message_basis must have shape {(H, rank, D)}, got {tuple(message_basis.shape)}")
        if rank > 64:
            raise ValueError(f"the HIP kernel only supports low-rank features <= 64, got {rank}")
        ext.message = tuple(_on_device(n, t, dev, s).float().contiguous() for n, t, s in (
            ("message_left", message_left, (B, H, N, N, rank)), ("message_right", message_right, (B, H, N, N, rank)),
            ("message_basis", message_basis, (H, rank, D))))
    return ext


def _operand_views(q, k1, v1, k2, v2, cdt, excluded: bool):
    """The (q, k/v) {batch, head, token} element strides when the five [B, H, N, D] operands can be read
    in place by the pair kernel (views such as the chunks of an in_proj output), else None (the operands
    are then copied to the contiguous layout).  The pair kernel takes 16-bit operands already in the
    compute dtype, head_dim <= 64 and a multiple of 8, tokens <= 512, no pair_valid and no angle or message
    term (`excluded`), unit-stride d, strides that are multiples of 8 elements below 2^31 and 16-byte
    aligned bases; k1, v1, k2 and v2 share strides."""
    B, H, N, D = q.shape
    if excluded or cdt not in (torch.float16, torch.bfloat16) or D % 8 != 0 or D > 64 or N > 512:
        return None
    ts = (q, k1, v1, k2, v2)
    if all(t.is_contiguous() for t in ts):
        return None
    if any(t.dtype != cdt or t.stride(3) != 1 or t.data_ptr() % 16 != 0 for t in ts):
        return None
    qs = tuple(q.stride()[:3])
    kvs = tuple(k1.stride()[:3])
    if any(tuple(t.stride()[:3]) != kvs for t in (v1, k2, v2)):
        return None
    if any(x < 0 or x % 8 != 0 or x >= 2**31 for x in qs + kvs + (N * H * D, H * D)):
        return None
    return qs, kvs


def hip_simplicial_attention_forward(
    q: torch.Tensor,
    k1: torch.Tensor,
    v1: torch.Tensor,
    k2: torch.Tensor,
    v2: torch.Tensor,
    *,
    query_valid: torch.Tensor,
    pair_key_valid: torch.Tensor,
    pair_valid: torch.Tensor | None,
    u: torch.Tensor | None = None,
    v_bias: torch.Tensor | None = None,
    w: torch.Tensor | None = None,
    gate: torch.Tensor | None = None,
    angle_left: torch.Tensor | None = None,
    angle_right: torch.Tensor | None = None,
    angle_gate: torch.Tensor | None = None,
    message_left: torch.Tensor | None = None,
    message_right: torch.Tensor | None = None,
    message_basis: torch.Tensor | None = None,
    precision: str = "bf16_tc",
    need_backward_state: bool = True,
) -> tuple[torch.Tensor, torch.Tensor | None, torch.Tensor | None]:
    """Returns ``(out[q.dtype] (B,H,N,D), lse fp32 (B,H,N), out fp32 (B,H,N,D))``.

    With ``need_backward_state=False`` (inference) only ``out`` is produced and
    the other two are None, which skips the fp32 output and lse writes.
    """
    if not HIP_AVAILABLE:
        raise RuntimeError(f"HIP simplicial attention is unavailable: {_native.load_error()}")
    if q.device.type != "cuda":
        raise RuntimeError("hip_simplicial_attention_forward requires GPU tensors")
    precision = normalize_simplicial_precision(precision)
    if q.dim() != 4:
        raise ValueError(f"q must have shape (B, H, N, D), got {tuple(q.shape)}")
    B, H, N, D = q.shape
    for name, t in (("k1", k1), ("v1", v1), ("k2", k2), ("v2", v2)):
        if t.shape != q.shape:
            raise ValueError(f"{name} must have shape {tuple(q.shape)}, got {tuple(t.shape)}")
        if t.device != q.device:
            raise RuntimeError(f"{name} must be on {q.device}")
    if tuple(query_valid.shape) != (B, N) or tuple(pair_key_valid.shape) != (B, N):
        raise ValueError(f"query_valid and pair_key_valid must have shape {(B, N)}")
    if pair_valid is not None and tuple(pair_valid.shape) != (B, N, N):
        raise ValueError(f"pair_valid must have shape {(B, N, N)}, got {tuple(pair_valid.shape)}")
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise RuntimeError(f"the HIP backend only supports float16/bfloat16/float32 inputs, got {q.dtype}")

    cdt = _compute_dtype(q.dtype, precision)
    views = _operand_views(q, k1, v1, k2, v2, cdt,
                           angle_left is not None or message_left is not None or pair_valid is not None)
    if views is not None:
        ops = [q, k1, v1, k2, v2]
        q_stride, kv_stride = views
    else:
        ops = [t.to(device=q.device, dtype=cdt).contiguous() for t in (q, k1, v1, k2, v2)]
        q_stride = kv_stride = (0, 0, 0)
    qv = query_valid.to(device=q.device, dtype=torch.bool).contiguous()
    pkv = pair_key_valid.to(device=q.device, dtype=torch.bool).contiguous()
    pv = None if pair_valid is None else pair_valid.to(device=q.device, dtype=torch.bool).contiguous()

    out_direct = q.dtype == cdt
    out_stride = (0, 0, 0)
    if views is not None:
        # written in the merged [B, N, H, D] layout that _merge_heads / out_proj read, returned as its
        # [B, H, N, D] view
        out = torch.empty((B, N, H, D), device=q.device, dtype=q.dtype).permute(0, 2, 1, 3)
        out_stride = (N * H * D, D, H * D)
    else:
        out = torch.empty((B, H, N, D), device=q.device, dtype=q.dtype) if out_direct else None
    out_f32 = None
    if need_backward_state or not out_direct:
        out_f32 = torch.empty((B, H, N, D), device=q.device, dtype=torch.float32)
    lse = torch.empty((B, H, N), device=q.device, dtype=torch.float32) if need_backward_state else None

    ext = _prepare_extras(q, B, H, N, D, u, v_bias, w, gate, angle_left, angle_right, angle_gate,
                          message_left, message_right, message_basis)

    lib = _native.lib()
    # (the factorized bias alone runs in the pair kernel and uses the workspace too)
    ws_bytes = lib.mf_simplicial_fwd_workspace_size(B, H, N, D, _native.dtype_code(cdt))
    ws = _native.workspace(ws_bytes, q.device)
    args = _native.MfSimplicialFwdArgs(
        q=ops[0].data_ptr(), k1=ops[1].data_ptr(), v1=ops[2].data_ptr(),
        k2=ops[3].data_ptr(), v2=ops[4].data_ptr(),
        query_valid=qv.data_ptr(), pair_key_valid=pkv.data_ptr(),
        pair_valid=None if pv is None else pv.data_ptr(),
        out=None if out is None else out.data_ptr(),
        out_f32=None if out_f32 is None else out_f32.data_ptr(),
        lse=None if lse is None else lse.data_ptr(),
        workspace=None if ws is None else ws.data_ptr(), workspace_bytes=ws_bytes,
        batch=B, heads=H, tokens=N, head_dim=D,
        dtype=_native.dtype_code(cdt), precision=_native.MF_PREC[precision],
        q_stride=(ctypes.c_int64 * 3)(*q_stride), kv_stride=(ctypes.c_int64 * 3)(*kv_stride),
        out_stride=(ctypes.c_int64 * 3)(*out_stride),
        **ext.fields(),
    )
    with torch.cuda.device(q.device):
        status = lib.mf_simplicial_fwd(args, _native.current_stream(q.device))
    _native.check(status, "mf_simplicial_fwd")
    if out is None:
        out = out_f32.to(q.dtype)
    if not need_backward_state:
        return out, None, None
    return out, lse, out_f32


def hip_simplicial_attention_backward(
    grad_out: torch.Tensor,
    q: torch.Tensor,
    k1: torch.Tensor,
    v1: torch.Tensor,
    k2: torch.Tensor,
    v2: torch.Tensor,
    out: torch.Tensor,
    lse: torch.Tensor,
    *,
    query_valid: torch.Tensor,
    pair_key_valid: torch.Tensor,
    pair_valid: torch.Tensor | None,
    u: torch.Tensor | None = None,
    v_bias: torch.Tensor | None = None,
    w: torch.Tensor | None = None,
    gate: torch.Tensor | None = None,
    angle_left: torch.Tensor | None = None,
    angle_right: torch.Tensor | None = None,
    angle_gate: torch.Tensor | None = None,
    message_left: torch.Tensor | None = None,
    message_right: torch.Tensor | None = None,
    message_basis: torch.Tensor | None = None,
    precision: str = "bf16_tc",
    need_du: bool = True,
    need_dv_bias: bool = True,
    need_dw: bool = True,
    need_dgate: bool = True,
    need_dangle_left: bool = True,
    need_dangle_right: bool = True,
    need_dangle_gate: bool = True,
    need_dmessage_left: bool = True,
    need_dmessage_right: bool = True,
    need_dmessage_basis: bool = True,
):
    """Returns the 15-tuple of triton_simplicial_attention.py:963-979 (None for grads not needed or absent).

    The gradients come from the deterministic HIP entry point ``mf_simplicial_bwd``
    (bitwise reproducible; bf16 MFMA for bf16 operands without angle / message
    terms, rounding the score products to bf16 as the reference's backward rounds
    them to the input type and carrying the value products as bf16 hi + lo; fp32
    MFMA for fp32 and fp16 operands and for every call with low-rank angle or
    message terms, whose gradients -- dangle_left/right/gate, dmessage_left/right/
    basis, triton_simplicial_attention.py:488-515,575-782 -- the kernel computes
    too).  Shapes beyond that kernel's LDS capacity (the library reports them)
    recompute the forward with the fp32-core torch path on the same device and
    take its autograd gradients -- the reference's own ``debug_torch_backward``
    route (simplicial_attention.py:454-552).  ``last_backward_impl`` records which
    of the two ran ("hip" or "torch_recompute").
    """
    global last_backward_impl
    flags = dict(need_du=need_du, need_dv_bias=need_dv_bias, need_dw=need_dw, need_dgate=need_dgate,
                 need_dangle_left=need_dangle_left, need_dangle_right=need_dangle_right,
                 need_dangle_gate=need_dangle_gate, need_dmessage_left=need_dmessage_left,
                 need_dmessage_right=need_dmessage_right, need_dmessage_basis=need_dmessage_basis)
    result = _kernel_backward(grad_out, q, k1, v1, k2, v2, out, lse, query_valid, pair_key_valid, pair_valid,
                              u, v_bias, w, gate, angle_left, angle_right, angle_gate, message_left, message_right,
                              message_basis, flags)
    if result is not None:
        last_backward_impl = "hip"
        return result
    last_backward_impl = "torch_recompute"
    return _recompute_backward(grad_out, q, k1, v1, k2, v2, query_valid=query_valid,
                               pair_key_valid=pair_key_valid, pair_valid=pair_valid, u=u, v_bias=v_bias, w=w,
                               gate=gate, angle_left=angle_left, angle_right=angle_right, angle_gate=angle_gate,
                               message_left=message_left, message_right=message_right,
                               message_basis=message_basis, **flags)


last_backward_impl: str | None = None


def _kernel_backward(grad_out, q, k1, v1, k2, v2, out, lse, query_valid, pair_key_valid, pair_valid,
                     u, v_bias, w, gate, angle_left, angle_right, angle_gate, message_left, message_right,
                     message_basis, flags):
    """mf_simplicial_bwd; None when the library reports the shape as beyond its capacity."""
    if not HIP_AVAILABLE:
        raise RuntimeError(f"HIP simplicial attention is unavailable: {_native.load_error()}")
    if q.device.type != "cuda":
        raise RuntimeError("hip_simplicial_attention_backward requires GPU tensors")
    B, H, N, D = q.shape
    dev = q.device
    dt = q.dtype if q.dtype in (torch.float16, torch.bfloat16, torch.float32) else torch.float32
    ops = [t.to(device=dev, dtype=dt).contiguous() for t in (q, k1, v1, k2, v2)]
    gdt = grad_out.dtype if grad_out.dtype in (torch.float16, torch.bfloat16, torch.float32) else torch.float32
    go = grad_out.to(device=dev, dtype=gdt).contiguous()
    out32 = out.to(device=dev, dtype=torch.float32).contiguous()
    lse32 = lse.to(device=dev, dtype=torch.float32).contiguous()
    for name, t, shape in (("grad_out", go, (B, H, N, D)), ("out", out32, (B, H, N, D)), ("lse", lse32, (B, H, N))):
        if tuple(t.shape) != shape:
            raise ValueError(f"{name} must have shape {shape}, got {tuple(t.shape)}")
    qv = query_valid.to(device=dev, dtype=torch.bool).contiguous()
    pkv = pair_key_valid.to(device=dev, dtype=torch.bool).contiguous()
    pv = None if pair_valid is None else pair_valid.to(device=dev, dtype=torch.bool).contiguous()
    if tuple(qv.shape) != (B, N) or tuple(pkv.shape) != (B, N) or (pv is not None and tuple(pv.shape) != (B, N, N)):
        raise ValueError("query_valid / pair_key_valid must be (B, N) and pair_valid (B, N, N)")
    ext = _prepare_extras(q, B, H, N, D, u, v_bias, w, gate, angle_left, angle_right, angle_gate,
                          message_left, message_right, message_basis)
    # bf16 operands, grad_out and leaves (bias terms included), no low-rank term: the library writes every
    # element of bf16 gradients (no fill, no cast); otherwise fp32 gradients, zero-filled here and cast to the
    # leaves' dtypes
    g16 = (dt == torch.bfloat16 and gdt == torch.bfloat16 and ext.angle is None and ext.message is None
           and D % 8 == 0 and N <= 4096 and all(t.dtype == torch.bfloat16 for t in (q, k1, v1, k2, v2))
           and (ext.bias is None or all(t.dtype == torch.bfloat16 for t in (u, v_bias, w, gate))))
    if g16:
        grads = [torch.empty(B, H, N, D, device=dev, dtype=torch.bfloat16) for _ in range(5)]
    else:
        grads = [torch.zeros(B, H, N, D, device=dev, dtype=torch.float32) for _ in range(5)]
    bias_grads = [None] * 4
    if ext.bias is not None:
        for idx, (name, shape) in enumerate((("need_du", (B, H, N, N)), ("need_dv_bias", (B, H, N, N)),
                                             ("need_dw", (B, H, N, N)), ("need_dgate", (B, H, N)))):
            if flags[name]:
                bias_grads[idx] = (torch.empty(shape, device=dev, dtype=torch.bfloat16) if g16 else
                                   torch.zeros(shape, device=dev, dtype=torch.float32))
    # low-rank gradients: (dangle_left, dangle_right, dangle_gate), (dmessage_left, dmessage_right, dmessage_basis)
    lr_grads: list[torch.Tensor | None] = [None] * 6
    if ext.angle is not None:
        ra = int(ext.angle[0].shape[-1])
        for idx, (name, shape) in enumerate((("need_dangle_left", (B, H, N, N, ra)),
                                             ("need_dangle_right", (B, H, N, N, ra)),
                                             ("need_dangle_gate", (B, H, N)))):
            if flags[name]:
                lr_grads[idx] = torch.zeros(shape, device=dev, dtype=torch.float32)
    rm = 0
    if ext.message is not None:
        rm = int(ext.message[0].shape[-1])
        for idx, (name, shape) in enumerate((("need_dmessage_left", (B, H, N, N, rm)),
                                             ("need_dmessage_right", (B, H, N, N, rm)),
                                             ("need_dmessage_basis", (H, rm, D)))):
            if flags[name]:
                lr_grads[3 + idx] = torch.zeros(shape, device=dev, dtype=torch.float32)
    # the message term's coefficients, or the pair kernel's plan and partial sums (bf16, head_dim 64)
    nbytes = int(_native.lib().mf_simplicial_bwd_workspace_size(B, H, N, D, rm))
    workspace = torch.empty(nbytes, device=dev, dtype=torch.uint8) if nbytes > 0 else None
    f = ext.fields()
    args = _native.MfSimplicialBwdArgs(
        q=ops[0].data_ptr(), k1=ops[1].data_ptr(), v1=ops[2].data_ptr(), k2=ops[3].data_ptr(), v2=ops[4].data_ptr(),
        grad_out=go.data_ptr(), out=out32.data_ptr(), lse=lse32.data_ptr(), query_valid=qv.data_ptr(),
        pair_key_valid=pkv.data_ptr(), pair_valid=None if pv is None else pv.data_ptr(),
        bias_u=f.get("bias_u"), bias_v=f.get("bias_v"), bias_w=f.get("bias_w"), bias_gate=f.get("bias_gate"),
        bias_dtype=f.get("bias_dtype", 0), grad_dtype=_native.dtype_code(gdt),
        dq=grads[0].data_ptr(), dk1=grads[1].data_ptr(), dv1=grads[2].data_ptr(), dk2=grads[3].data_ptr(),
        dv2=grads[4].data_ptr(), du=_native.ptr(bias_grads[0]), dv_bias=_native.ptr(bias_grads[1]),
        dw=_native.ptr(bias_grads[2]), dgate=_native.ptr(bias_grads[3]),
        batch=B, heads=H, tokens=N, head_dim=D, dtype=_native.dtype_code(dt),
        grads_dtype=_native.dtype_code(torch.bfloat16 if g16 else torch.float32),
        angle_rank=f.get("angle_rank", 0), message_rank=f.get("message_rank", 0),
        angle_left=f.get("angle_left"), angle_right=f.get("angle_right"), angle_gate=f.get("angle_gate"),
        message_left=f.get("message_left"), message_right=f.get("message_right"),
        message_basis=f.get("message_basis"),
        dangle_left=_native.ptr(lr_grads[0]), dangle_right=_native.ptr(lr_grads[1]),
        dangle_gate=_native.ptr(lr_grads[2]), dmessage_left=_native.ptr(lr_grads[3]),
        dmessage_right=_native.ptr(lr_grads[4]), dmessage_basis=_native.ptr(lr_grads[5]),
        workspace=_native.ptr(workspace), workspace_bytes=0 if workspace is None else workspace.numel())
    lib = _native.lib()
    with torch.cuda.device(dev):
        status = lib.mf_simplicial_bwd(args, _native.current_stream(dev))
    if status == _native.MF_ERR_UNSUPPORTED:
        return None
    _native.check(status, "mf_simplicial_bwd")
    core = grads if g16 else [g.to(t.dtype) for g, t in zip(grads, (q, k1, v1, k2, v2))]
    optional = [None] * 10
    if ext.bias is not None:
        for idx, src in enumerate((u, v_bias, w, gate)):
            if bias_grads[idx] is not None:
                optional[idx] = bias_grads[idx] if g16 else bias_grads[idx].to(src.dtype)
    for idx, src in enumerate((angle_left, angle_right, angle_gate, message_left, message_right, message_basis)):
        if lr_grads[idx] is not None:
            optional[4 + idx] = lr_grads[idx].to(src.dtype)
    return (*core, *optional)


def _recompute_backward(
    grad_out, q, k1, v1, k2, v2, *, query_valid, pair_key_valid, pair_valid, u, v_bias, w, gate,
    angle_left, angle_right, angle_gate, message_left, message_right, message_basis,
    need_du, need_dv_bias, need_dw, need_dgate, need_dangle_left, need_dangle_right, need_dangle_gate,
    need_dmessage_left, need_dmessage_right, need_dmessage_basis,
):
    """fp32-core torch recompute + autograd on the inputs' device (simplicial_attention.py:454-552)."""
    has_bias = u is not None
    has_angle = angle_left is not None
    has_message = message_left is not None
    leaves = [t.detach().requires_grad_(True) for t in (q, k1, v1, k2, v2)]
    opt: list[torch.Tensor | None] = [None] * 10
    if has_bias:
        opt[0:4] = [t.detach().requires_grad_(True) for t in (u, v_bias, w, gate)]
    if has_angle:
        opt[4:7] = [t.detach().requires_grad_(True) for t in (angle_left, angle_right, angle_gate)]
    if has_message:
        opt[7:10] = [t.detach().requires_grad_(True) for t in (message_left, message_right, message_basis)]
    with torch.enable_grad():
        fb = SimplicialFactorizedBias(u=opt[0], v=opt[1], w=opt[2], gate=opt[3]) if has_bias else None
        ar = SimplicialLowRankAngleResidual(left=opt[4], right=opt[5], gate=opt[6]) if has_angle else None
        mr = SimplicialLowRankMessageResidual(left=opt[7], right=opt[8]) if has_message else None
        mask = SimplicialAttentionMask(query_valid=query_valid, pair_key_valid=pair_key_valid, pair_valid=pair_valid)
        ref = simplicial_attention_torch_from_projected(
            *leaves, attention_mask=mask, factorized_bias=fb, angle_residual=ar, message_residual=mr,
            message_basis=opt[9] if has_message else None, chunk_size=128, fp32_core=True,
        )
        inputs = leaves + [t for t in opt if t is not None]
        grads = list(torch.autograd.grad(ref, inputs, grad_out.to(ref.dtype), allow_unused=True))
    core = grads[:5]
    rest = grads[5:]
    flags = [need_du, need_dv_bias, need_dw, need_dgate, need_dangle_left, need_dangle_right,
             need_dangle_gate, need_dmessage_left, need_dmessage_right, need_dmessage_basis]
    optional: list[torch.Tensor | None] = []
    cursor = 0
    for present, group in ((has_bias, range(0, 4)), (has_angle, range(4, 7)), (has_message, range(7, 10))):
        for idx in group:
            if present:
                g = rest[cursor]
                cursor += 1
                optional.append(g if flags[idx] else None)
            else:
                optional.append(None)
    return (*core, *optional)


# Reference names.
triton_simplicial_attention_forward = hip_simplicial_attention_forward
triton_simplicial_attention_backward = hip_simplicial_attention_backward
