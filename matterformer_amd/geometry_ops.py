"""Geometry kernels of the hot path: kNN top-k, radius (cutoff) masks and
radius (local) attention, each one launch of a gfx950 kernel through the C ABI
(include/mf_capi.h).

The reference has no fused kernels for these; the conventions come from its
geometry adapters and attention modules:

  knn_graph          pair distance of NonPeriodicGeometryAdapter.forward
                     (src/matterformer/geometry/adapters.py:98-100); the
                     neighbour list the legacy knn / knn_graph built with
                     cdist + topk (legacy/rapidash_v5/models/rapidash_utils.py:139-193),
                     here with ties ordered by index.
  lattice_terms      lattice_latent_to_gram, lattice_latent_to_y1 and the periodic adapter's
                     cell scale (src/matterformer/geometry/lattice.py:12-131, adapters.py:173-192);
                     lattice_to_gram is its first output.
  radius_mask        minimum-image distance of PeriodicGeometryAdapter.forward
                     (adapters.py:141-149,176-190) or the plain distance
                     (:98-99), thresholded at a cutoff, as bits.
  radius_attention   masked attention through an additive mask
                     (src/matterformer/models/transformer.py:256-268,
                     src/matterformer/models/regular_attention.py:262-268,303-308).

Inputs must be CUDA (ROCm) tensors; nothing here falls back to another
implementation: a missing library or a CPU tensor raises RuntimeError.
"""

from __future__ import annotations

import math

import torch

from matterformer_amd import _native

MASK_BLOCK = 64  # the tile of radius_attention; radius_mask's default block


def _require_device(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError("matterformer_amd geometry ops need CUDA (ROCm) tensors")
        if t.device != dev:
            raise RuntimeError("all tensors must be on the same device")
    return dev


def _pad_bytes(pad_mask: torch.Tensor | None, B: int, N: int) -> torch.Tensor | None:
    if pad_mask is None:
        return None
    if pad_mask.shape != (B, N):
        raise ValueError(f"pad_mask must have shape ({B}, {N}), got {tuple(pad_mask.shape)}")
    return pad_mask.to(torch.uint8).contiguous()


def knn_graph(coords: torch.Tensor, k: int, pad_mask: torch.Tensor | None = None, *,
              exclude_self: bool = True, return_dist: bool = True):
    """k nearest valid neighbours of every atom.

    coords (B, N, 3); pad_mask (B, N) bool, True = padding (the reference's
    key_padding_mask convention).  Returns idx int32 (B, N, k), ascending by
    (d^2, j), -1 where fewer than k candidates exist and for padded atoms,
    and dist fp32 (B, N, k) (+inf in the same places) when return_dist.
    """
    if coords.ndim != 3 or coords.shape[-1] != 3:
        raise ValueError(f"coords must have shape (B, N, 3), got {tuple(coords.shape)}")
    if not 1 <= int(k) <= 64:
        raise ValueError(f"k must be in [1, 64], got {k}")
    dev = _require_device(coords, pad_mask)
    B, N, _ = coords.shape
    c = coords.float().contiguous()
    pad = _pad_bytes(pad_mask, B, N)
    idx = torch.empty(B, N, int(k), dtype=torch.int32, device=dev)
    dist = torch.empty(B, N, int(k), dtype=torch.float32, device=dev) if return_dist else None
    args = _native.MfKnnArgs(
        coords=c.data_ptr(), pad_mask=_native.ptr(pad), idx=idx.data_ptr(), dist=_native.ptr(dist),
        batch=B, atoms=N, k=int(k), exclude_self=int(bool(exclude_self)))
    with torch.cuda.device(dev):
        _native.check(_native.lib().mf_knn(args, _native.current_stream(dev)), "mf_knn")
    return (idx, dist) if return_dist else idx


def knn_mask(idx: torch.Tensor, pad_mask: torch.Tensor | None = None, *, include_self: bool = True,
             with_block_mask: bool = True):
    """Local-attention masks from kNN lists: mask[b, i, j] = valid_i and (j in idx[b, i] or j == i).

    idx (B, N, k) int32 as knn_graph returns it (-1 = none); pad_mask (B, N) bool, True = padding.
    Returns mask_bits int32 (B, N, ceil(N/32)) and, with with_block_mask, block_mask uint8
    (B, ceil(N/64), ceil(N/64)) -- the layout radius_attention reads.  The reference's trunk can only
    express such a mask as a 0 / -inf attn_head_bias (transformer.py:256-268); these are its allowed entries.
    """
    if idx.ndim != 3 or idx.dtype != torch.int32:
        raise ValueError(f"idx must be int32 of shape (B, N, k), got {idx.dtype} {tuple(idx.shape)}")
    dev = _require_device(idx, pad_mask)
    B, N, K = idx.shape
    pad = _pad_bytes(pad_mask, B, N)
    W = (N + 31) // 32
    NB = (N + MASK_BLOCK - 1) // MASK_BLOCK
    bits = torch.empty(B, N, W, dtype=torch.int32, device=dev)
    blocks = torch.empty(B, NB, NB, dtype=torch.uint8, device=dev) if with_block_mask else None
    ic = idx.contiguous()
    args = _native.MfKnnMaskArgs(idx=ic.data_ptr(), pad_mask=_native.ptr(pad), mask_bits=bits.data_ptr(),
                                 block_mask=_native.ptr(blocks), batch=B, atoms=N, k=K,
                                 include_self=int(bool(include_self)))
    with torch.cuda.device(dev):
        _native.check(_native.lib().mf_knn_mask(args, _native.current_stream(dev)), "mf_knn_mask")
    return (bits, blocks) if with_block_mask else bits


def _lattice_terms_torch(lat: torch.Tensor, rep: str):
    """The torch formulation (CPU tensors): lattice_latent_to_gram, lattice_latent_to_y1
    (src/matterformer/geometry/lattice.py:12-131) and the periodic adapter's cell scale
    (adapters.py:192)."""
    B = lat.shape[0]
    cell = torch.zeros(B, 3, 3, device=lat.device, dtype=lat.dtype)
    if rep == "y1":
        lengths = torch.exp(lat[:, :3].clamp(min=-5.0, max=5.0))
        ca, cb, cg = lat[:, 3:].clamp(min=-0.9999, max=0.9999).unbind(dim=-1)
        sg = torch.sqrt((1.0 - cg.square()).clamp_min(1e-8))
        cell[:, 0, 0] = lengths[:, 0]
        cell[:, 1, 0] = lengths[:, 1] * cg
        cell[:, 1, 1] = lengths[:, 1] * sg
        cell[:, 2, 0] = lengths[:, 2] * cb
        cell[:, 2, 1] = lengths[:, 2] * (ca - cb * cg) / sg
        cell[:, 2, 2] = torch.sqrt(lengths[:, 2].square() - cell[:, 2, 0].square()
                                   - cell[:, 2, 1].square()).clamp_min(1e-8)
    else:
        diag = torch.exp(lat[:, [0, 2, 5]].clamp(min=-5.0, max=5.0))
        off = lat[:, [1, 3, 4]].clamp(min=-10.0, max=10.0)
        cell[:, 0, 0] = diag[:, 0]
        cell[:, 1, 0] = off[:, 0]
        cell[:, 1, 1] = diag[:, 1]
        cell[:, 2, 0] = off[:, 1]
        cell[:, 2, 1] = off[:, 2]
        cell[:, 2, 2] = diag[:, 2]
    gram = torch.nan_to_num(torch.matmul(cell, cell.transpose(-1, -2)), nan=0.0, posinf=0.0, neginf=0.0)
    if rep == "y1":
        y1 = torch.cat([lat[:, :3].clamp(min=-5.0, max=5.0), lat[:, 3:].clamp(min=-0.9999, max=0.9999)], dim=-1)
    else:
        lengths = torch.sqrt(torch.diagonal(gram, dim1=-2, dim2=-1).clamp_min(1e-8))
        den_a = (lengths[:, 1] * lengths[:, 2]).clamp_min(1e-8)
        den_b = (lengths[:, 0] * lengths[:, 2]).clamp_min(1e-8)
        den_g = (lengths[:, 0] * lengths[:, 1]).clamp_min(1e-8)
        cos = torch.stack([(gram[:, 1, 2] / den_a), (gram[:, 0, 2] / den_b), (gram[:, 0, 1] / den_g)], dim=-1)
        y1 = torch.cat([torch.log(lengths.clamp_min(1e-8)), cos.clamp(min=-0.9999, max=0.9999)], dim=-1)
    cell_scale = torch.exp(y1[:, :3]).mean(dim=-1).clamp_min(1e-8)
    return gram, y1, cell_scale


def lattice_terms(lattice: torch.Tensor, lattice_repr: str = "y1"):
    """(gram (B, 3, 3), y1 (B, 6), cell_scale (B,)) of lattice latents (B, 6), fp32: the metric
    C C^T of lattice_latent_to_gram (src/matterformer/geometry/lattice.py:12-59,94-100), the y1
    latent of lattice_latent_to_y1 (:65-91,103-131) and the periodic adapter's cell scale
    max(mean(exp(y1[:, :3])), 1e-8) (adapters.py:173-174,192).  CUDA tensors: one
    mf_lattice_terms launch; CPU tensors: the torch formulation."""
    lat = lattice.float()
    if lat.ndim != 2 or lat.shape[-1] != 6:
        raise ValueError(f"lattice must have shape (B, 6), got {tuple(lat.shape)}")
    rep = lattice_repr.lower()
    if rep not in ("y1", "ltri"):
        raise ValueError(f"Unsupported lattice_repr: {lattice_repr}")
    if lat.device.type != "cuda":
        return _lattice_terms_torch(lat, rep)
    dev = lat.device
    B = lat.shape[0]
    lat = lat.contiguous()
    gram = torch.empty(B, 3, 3, device=dev, dtype=torch.float32)
    y1 = torch.empty(B, 6, device=dev, dtype=torch.float32)
    scale = torch.empty(B, device=dev, dtype=torch.float32)
    code = _native.MF_LATTICE_Y1 if rep == "y1" else _native.MF_LATTICE_LTRI
    with torch.cuda.device(dev):
        _native.check(_native.lib().mf_lattice_terms(lat.data_ptr(), B, code, gram.data_ptr(), y1.data_ptr(),
                                                     scale.data_ptr(), _native.current_stream(dev)),
                      "mf_lattice_terms")
    return gram, y1, scale


def lattice_to_gram(lattice: torch.Tensor, lattice_repr: str = "y1") -> torch.Tensor:
    """Metric G = cell cell^T of a lattice latent (B, 6), as lattice_latent_to_gram
    (src/matterformer/geometry/lattice.py:12-59,94-100): lower-triangular cell
    with a along x and b in the xy plane, in fp32 (non-finite entries 0)."""
    return lattice_terms(lattice, lattice_repr)[0]


def radius_mask(coords: torch.Tensor, cutoff: float, *, gram: torch.Tensor | None = None,
                lattice: torch.Tensor | None = None, lattice_repr: str = "y1",
                pad_mask: torch.Tensor | None = None, pbc_radius: int = 1, block: int = MASK_BLOCK,
                with_block_mask: bool = True):
    """Neighbour mask d(i, j) <= cutoff as bits.

    Periodic when ``gram`` (B, 3, 3) or ``lattice`` (B, 6) is given: coords are
    fractional and d is the minimum-image distance over the offsets
    {-pbc_radius..pbc_radius}^3.  Returns mask_bits int32 (B, N, ceil(N/32))
    (bit t of word w = column 32 w + t; the bit pattern is the kernel's uint32)
    and block_mask uint8 (B, NB, NB) (or None).
    """
    if coords.ndim != 3 or coords.shape[-1] != 3:
        raise ValueError(f"coords must have shape (B, N, 3), got {tuple(coords.shape)}")
    if gram is not None and lattice is not None:
        raise ValueError("pass gram or lattice, not both")
    if lattice is not None:
        gram = lattice_to_gram(lattice, lattice_repr)
    if gram is not None and pbc_radius not in (1, 2):
        raise ValueError(f"pbc_radius must be 1 or 2, got {pbc_radius}")
    dev = _require_device(coords, gram, pad_mask)
    B, N, _ = coords.shape
    c = coords.float().contiguous()
    g = None if gram is None else gram.float().contiguous()
    if g is not None and g.shape != (B, 3, 3):
        raise ValueError(f"gram must have shape ({B}, 3, 3), got {tuple(g.shape)}")
    pad = _pad_bytes(pad_mask, B, N)
    W = (N + 31) // 32
    NB = (N + block - 1) // block
    bits = torch.empty(B, N, W, dtype=torch.int32, device=dev)
    blocks = torch.empty(B, NB, NB, dtype=torch.uint8, device=dev) if with_block_mask else None
    args = _native.MfRadiusMaskArgs(
        coords=c.data_ptr(), gram=_native.ptr(g), pad_mask=_native.ptr(pad), mask_bits=bits.data_ptr(),
        block_mask=_native.ptr(blocks), cutoff=float(cutoff), batch=B, atoms=N, block=int(block),
        pbc_radius=int(pbc_radius))
    with torch.cuda.device(dev):
        _native.check(_native.lib().mf_radius_mask(args, _native.current_stream(dev)), "mf_radius_mask")
    return bits, blocks


def radius_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask_bits: torch.Tensor,
                     block_mask: torch.Tensor | None = None, *, scale: float | None = None,
                     return_lse: bool = False, return_fp32: bool = False):
    """softmax_j(scale q_i . k_j over the neighbours j of i) v_j.

    q, k, v (B, H, N, D) bf16/fp16 with D in {32, 64, 128}; mask_bits from
    radius_mask; block_mask from radius_mask with block=64 (or None: every
    tile is visited).  Rows without a neighbour are 0 (lse 0).  Returns out in
    q's dtype, plus lse (B, H, N) fp32 and/or the fp32 output when asked.
    """
    if q.ndim != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError("q, k, v must share the shape (B, H, N, D)")
    if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise RuntimeError("radius_attention only supports float16/bfloat16 q, k, v of one dtype")
    B, H, N, D = q.shape
    if D not in (32, 64, 128):
        raise RuntimeError(f"radius_attention supports head_dim 32, 64 or 128, got {D}")
    W = (N + 31) // 32
    if mask_bits.shape != (B, N, W) or mask_bits.dtype != torch.int32:
        raise ValueError(f"mask_bits must be int32 of shape ({B}, {N}, {W})")
    NB = (N + MASK_BLOCK - 1) // MASK_BLOCK
    if block_mask is not None and block_mask.shape != (B, NB, NB):
        raise ValueError(f"block_mask must have shape ({B}, {NB}, {NB}) (block {MASK_BLOCK})")
    dev = _require_device(q, k, v, mask_bits, block_mask)
    qc, kc, vc = q.contiguous(), k.contiguous(), v.contiguous()
    bits = mask_bits.contiguous()
    bm = None if block_mask is None else block_mask.to(torch.uint8).contiguous()
    out = torch.empty_like(qc)
    out32 = torch.empty(B, H, N, D, dtype=torch.float32, device=dev) if return_fp32 else None
    lse = torch.empty(B, H, N, dtype=torch.float32, device=dev) if return_lse else None
    s = float(D ** -0.5 if scale is None else scale)
    if not math.isfinite(s):
        raise ValueError("scale must be finite")
    args = _native.MfRadiusAttnArgs(
        q=qc.data_ptr(), k=kc.data_ptr(), v=vc.data_ptr(), mask_bits=bits.data_ptr(), block_mask=_native.ptr(bm),
        out=out.data_ptr(), out_f32=_native.ptr(out32), lse=_native.ptr(lse), scale=s, batch=B, heads=H, atoms=N,
        head_dim=D, dtype=_native.dtype_code(q.dtype))
    with torch.cuda.device(dev):
        _native.check(_native.lib().mf_radius_attn(args, _native.current_stream(dev)), "mf_radius_attn")
    result = (out,)
    if return_lse:
        result += (lse,)
    if return_fp32:
        result += (out32,)
    return result[0] if len(result) == 1 else result
