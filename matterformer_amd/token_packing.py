"""Valid atoms of a padded batch as the rows of one (T, C) matrix, and the per-token glue of the packed trunk.

The reference runs its AdaLN blocks on the padded (B, N, C) batch (transformer.py:296-316) and masks padded
atoms in attention.  Every valid row's result is independent of the padded rows, so the per-token work can
run on the T valid rows alone; only the attention kernels need a (B, H, W, D) head layout, here with the
molecules' valid atoms moved to the front (stable, so index order and kNN tie-breaks are kept) and
W = the largest valid count of the batch rather than the padded N.

On GPU tensors without autograd the glue runs on HIP kernels (token_rows.hip):
  mf_rows_to_heads   projections (T, P*H*D) -> (P, B, H, W, D), padded slots zero, q pre-scaled
  mf_heads_to_rows   attention output (B, H, W, D) -> (T, H*D)
  mf_adaln_rows      x' = x + gate * y and h = LN(x') * (1 + scale) + shift in one pass per row
and otherwise on the equivalent torch expressions (which autograd follows).
"""

from __future__ import annotations

import torch

from matterformer_amd import _native


def _native_ok(*tensors: torch.Tensor) -> bool:
    """HIP glue for GPU tensors when autograd does not follow the call (the kernels have no backward).  A
    missing library then raises (in _native.lib()) rather than falling back."""
    if not all(t.device.type == "cuda" for t in tensors):
        return False
    return not (torch.is_grad_enabled() and any(t.requires_grad for t in tensors))


def _aligned(*tensors: torch.Tensor) -> bool:
    return all(t.data_ptr() % 16 == 0 for t in tensors)


class TokenPacking:
    """The valid atoms (pad_mask False) of a padded batch.

    Row t of the packed matrix is atom ``rows[t] % N`` of molecule ``mol[t]`` (molecule-major, atom order
    kept); in the compact head layout it sits at position ``pos[t]`` of its molecule, whose valid atoms fill
    positions 0 .. count - 1 of ``width`` = max count.  Built once per batch (one host synchronisation for
    the sizes), so a HIP-graph capture of the trunk takes it as an argument.
    """

    def __init__(self, pad_mask: torch.Tensor) -> None:
        if pad_mask.ndim != 2:
            raise ValueError(f"pad_mask must have shape (B, N), got {tuple(pad_mask.shape)}")
        valid = ~pad_mask.bool()
        self.batch, self.atoms = (int(n) for n in pad_mask.shape)
        self.device = pad_mask.device
        counts = valid.sum(dim=1)
        sizes = torch.stack([counts.sum(), counts.max() if self.batch else counts.sum()]).cpu()
        self.tokens, self.width = int(sizes[0]), int(sizes[1])
        self.counts = counts
        self.rows = valid.reshape(-1).nonzero().squeeze(1)
        self.mol = torch.div(self.rows, self.atoms, rounding_mode="floor")
        self.pos = (valid.cumsum(dim=1) - 1).reshape(-1).index_select(0, self.rows)
        self.compact_rows = self.mol * self.width + self.pos
        self.mol32 = self.mol.to(torch.int32)
        self.compact_rows32 = self.compact_rows.to(torch.int32)
        slot = torch.full((self.batch * self.width,), -1, dtype=torch.int32, device=self.device)
        slot[self.compact_rows] = torch.arange(self.tokens, dtype=torch.int32, device=self.device)
        self.slot32 = slot
        self.compact_pad_mask = torch.arange(self.width, device=self.device)[None, :] >= counts[:, None]
        atom_index = torch.zeros(self.batch * self.width, dtype=torch.long, device=self.device)
        atom_index[self.compact_rows] = self.rows - self.mol * self.atoms
        self.atom_index = atom_index.view(self.batch, self.width)  # atom at each compact position (0 past count)

    # -- (B, N, ...) <-> packed rows -------------------------------------------------------------------------
    def pack(self, x: torch.Tensor) -> torch.Tensor:
        """(B, N, C) -> (T, C)."""
        return x.reshape(self.batch * self.atoms, x.shape[-1]).index_select(0, self.rows)

    def unpack(self, xp: torch.Tensor) -> torch.Tensor:
        """(T, C) -> (B, N, C), padded atoms zero."""
        out = xp.new_zeros(self.batch * self.atoms, xp.shape[-1])
        out.index_copy_(0, self.rows, xp)
        return out.view(self.batch, self.atoms, xp.shape[-1])

    def per_token(self, t: torch.Tensor) -> torch.Tensor:
        """(B, ...) per-molecule rows -> (T, ...)."""
        return t.index_select(0, self.mol)

    def compact(self, t: torch.Tensor) -> torch.Tensor:
        """(B, N, ...) -> (B, W, ...): each molecule's valid atoms first, zeros after."""
        tail = t.shape[2:]
        out = t.new_zeros((self.batch * self.width,) + tail)
        out[self.compact_rows] = t.reshape((self.batch * self.atoms,) + tail).index_select(0, self.rows)
        return out.view((self.batch, self.width) + tail)

    def compact_dims(self, t: torch.Tensor, *dims: int) -> torch.Tensor:
        """Atom axes ``dims`` of a (B, ...) tensor (bias terms, pair masks, gates) from N to the compact width W,
        each molecule's valid atoms first; positions past a molecule's count are zero (False)."""
        B, W = self.batch, self.width
        keep_all = ~self.compact_pad_mask
        for dim in dims:
            shape = [1] * t.ndim
            shape[0], shape[dim] = B, W
            full = list(t.shape)
            full[dim] = W
            t = t.gather(dim, self.atom_index.view(shape).expand(full))
            keep = keep_all.view(shape)
            t = t & keep if t.dtype == torch.bool else t.masked_fill(~keep, 0)
        return t

    # -- packed rows <-> compact head layout -----------------------------------------------------------------
    def to_heads(self, xp: torch.Tensor, parts: int, heads: int, head_dim: int, dtype: torch.dtype,
                 first_part_scale: float = 1.0) -> torch.Tensor:
        """(T, parts * heads * head_dim) -> (parts, B, heads, W, head_dim) in ``dtype``, empty slots zero;
        part 0 multiplied by first_part_scale in xp's dtype before the conversion."""
        if xp.shape != (self.tokens, parts * heads * head_dim):
            raise ValueError(f"projections must have shape ({self.tokens}, {parts * heads * head_dim})")
        out = torch.empty(parts, self.batch, heads, self.width, head_dim, dtype=dtype, device=xp.device)
        if _native_ok(xp) and head_dim % 8 == 0 and xp.is_contiguous() and _aligned(xp, out):
            args = _native.MfRowsToHeadsArgs(
                rows=xp.data_ptr(), slot=self.slot32.data_ptr(), heads=out.data_ptr(),
                first_part_scale=float(first_part_scale), tokens=self.tokens, parts=parts, batch=self.batch,
                heads_count=heads, width=self.width, head_dim=head_dim, src_dtype=_native.dtype_code(xp.dtype),
                dst_dtype=_native.dtype_code(dtype))
            with torch.cuda.device(xp.device):
                _native.check(_native.lib().mf_rows_to_heads(args, _native.current_stream(xp.device)),
                              "mf_rows_to_heads")
            return out
        src = xp.view(self.tokens, parts, heads, head_dim)
        if first_part_scale != 1.0:
            src = torch.cat([src[:, :1] * first_part_scale, src[:, 1:]], dim=1)
        out.zero_()
        out.permute(1, 3, 0, 2, 4)[self.mol, self.pos] = src.to(dtype)
        return out

    def from_heads(self, out: torch.Tensor, dtype: torch.dtype | None = None) -> torch.Tensor:
        """(B, H, W, D) attention output -> (T, H * D) in ``dtype`` (default: out's)."""
        B, H, W, D = out.shape
        if (B, W) != (self.batch, self.width):
            raise ValueError(f"attention output must have shape ({self.batch}, H, {self.width}, D)")
        dtype = out.dtype if dtype is None else dtype
        if _native_ok(out) and D % 8 == 0 and out.is_contiguous():
            rows = torch.empty(self.tokens, H * D, dtype=dtype, device=out.device)
            if _aligned(out, rows):
                args = _native.MfHeadsToRowsArgs(
                    heads=out.data_ptr(), row_index=self.compact_rows32.data_ptr(), rows=rows.data_ptr(),
                    tokens=self.tokens, batch=B, heads_count=H, width=W, head_dim=D,
                    src_dtype=_native.dtype_code(out.dtype), dst_dtype=_native.dtype_code(dtype))
                with torch.cuda.device(out.device):
                    _native.check(_native.lib().mf_heads_to_rows(args, _native.current_stream(out.device)),
                                  "mf_heads_to_rows")
                return rows
        return out.permute(0, 2, 1, 3)[self.mol, self.pos].reshape(self.tokens, H * D).to(dtype)


def adaln_rows(packing: TokenPacking, x: torch.Tensor, y: torch.Tensor | None = None,
               gate: torch.Tensor | None = None, shift: torch.Tensor | None = None,
               scale: torch.Tensor | None = None, *, eps: float = 1e-6, inplace: bool = False):
    """x' = x + gate[mol] * y (when y is given) and h = LN(x') * (1 + scale[mol]) + shift[mol] (when shift is
    given), LN without affine, each product and sum rounded to x's dtype as transformer.py:296-316's torch
    expressions are.  gate / shift / scale are (B, C) column slices of a block's ada_ln output.  Returns
    x', h or (x', h).  ``inplace`` lets the HIP path write x' over x."""
    if y is None and shift is None:
        raise ValueError("adaln_rows: nothing to compute")
    T, C = x.shape
    tensors = [t for t in (x, y, gate, shift, scale) if t is not None]
    native = (_native_ok(*tensors) and C % 8 == 0 and C <= 2048 and x.is_contiguous()
              and (y is None or y.is_contiguous()) and len({t.dtype for t in tensors}) == 1)
    mods = [t for t in (gate, shift, scale) if t is not None]
    if native:
        strides = {t.stride(0) for t in mods}
        native = (len(strides) == 1 and all(t.stride(1) == 1 for t in mods) and strides.pop() % 8 == 0
                  and _aligned(x, *mods, *([y] if y is not None else [])))
    if native:
        x_out = (x if inplace else torch.empty_like(x)) if y is not None else None
        h = torch.empty_like(x) if shift is not None else None
        args = _native.MfAdalnRowsArgs(
            x=x.data_ptr(), y=_native.ptr(y), gate=_native.ptr(gate), shift=_native.ptr(shift),
            scale=_native.ptr(scale), mol=packing.mol32.data_ptr(), x_out=_native.ptr(x_out), h_out=_native.ptr(h),
            eps=float(eps), tokens=T, channels=C, batch=packing.batch, mod_stride=mods[0].stride(0),
            dtype=_native.dtype_code(x.dtype))
        with torch.cuda.device(x.device):
            _native.check(_native.lib().mf_adaln_rows(args, _native.current_stream(x.device)), "mf_adaln_rows")
    else:
        x_out = x + packing.per_token(gate) * y if y is not None else None
        h = None
        if shift is not None:
            src = x_out if x_out is not None else x
            n = torch.nn.functional.layer_norm(src, (C,), eps=eps)
            h = n * packing.per_token(1.0 + scale) + packing.per_token(shift)
    if y is not None and shift is not None:
        return x_out, h
    return x_out if y is not None else h
