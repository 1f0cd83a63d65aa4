"""Radius (local) attention oracle -- TEST INFRASTRUCTURE ONLY.

The reference has no radius attention kernel; its only pairwise attention is
MHA with an additive mask, reached from the trunk through ``attn_head_bias``
(src/matterformer/models/transformer.py:256-268) and evaluated by
``nn.MultiheadAttention`` / ``F.scaled_dot_product_attention``
(src/matterformer/models/regular_attention.py:262-268,303-308).  With a
neighbour mask that is a dense masked softmax:

    out_i = sum_j softmax_j( scale * q_i . k_j  over j with mask[i,j] ) v_j

``masked_attention_fp64`` restates that in float64 (numpy).  Rows with no
allowed key (padding atoms) are 0, and their lse is 0.
Pinned by: torch's own ``F.scaled_dot_product_attention`` with a boolean mask
(an independent implementation) and the closed form for an all-equal-logit
row (mean of the allowed v_j), in tests/test_oracle_radius.py.
"""

from __future__ import annotations

import numpy as np


def masked_attention_fp64(q: np.ndarray, k: np.ndarray, v: np.ndarray, mask: np.ndarray, scale: float):
    """q,k,v (B,H,N,D); mask (B,N,N) bool -> (out (B,H,N,D), lse (B,H,N))."""
    q, k, v = (np.asarray(a, dtype=np.float64) for a in (q, k, v))
    B, H, N, D = q.shape
    s = np.einsum("bhid,bhjd->bhij", q, k) * scale
    m = mask[:, None, :, :]
    s = np.where(m, s, -np.inf)
    row_max = s.max(axis=-1, keepdims=True)
    has = np.isfinite(row_max)
    row_max = np.where(has, row_max, 0.0)
    p = np.where(m, np.exp(s - row_max), 0.0)
    tot = p.sum(axis=-1, keepdims=True)
    safe = np.where(tot > 0, tot, 1.0)
    out = np.einsum("bhij,bhjd->bhid", p / safe, v)
    lse = np.where(tot[..., 0] > 0, row_max[..., 0] + np.log(safe[..., 0]), 0.0)
    return out, lse


def lattice_y1_to_gram(y1: np.ndarray) -> np.ndarray:
    """y1 = [log a, log b, log c, cos alpha, cos beta, cos gamma] -> Gram matrix (B,3,3), float32.

    Lower-triangular cell of src/matterformer/geometry/lattice.py:32-47
    (a along x, b in the xy plane), G = cell cell^T (:94-100).
    """
    y1 = np.asarray(y1, dtype=np.float64)
    lengths = np.exp(np.clip(y1[:, :3], -5.0, 5.0))
    ca, cb, cg = np.clip(y1[:, 3:], -0.9999, 0.9999).T
    sg = np.sqrt(np.maximum(1.0 - cg * cg, 1e-8))
    cell = np.zeros((y1.shape[0], 3, 3))
    cell[:, 0, 0] = lengths[:, 0]
    cell[:, 1, 0] = lengths[:, 1] * cg
    cell[:, 1, 1] = lengths[:, 1] * sg
    cell[:, 2, 0] = lengths[:, 2] * cb
    cell[:, 2, 1] = lengths[:, 2] * (ca - cb * cg) / sg
    cell[:, 2, 2] = np.sqrt(np.maximum(lengths[:, 2] ** 2 - cell[:, 2, 0] ** 2 - cell[:, 2, 1] ** 2, 1e-16))
    return (cell @ cell.transpose(0, 2, 1)).astype(np.float32)
