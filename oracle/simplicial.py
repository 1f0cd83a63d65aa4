"""2-simplicial attention oracle (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py).

Two independent restatements:

``reference_path``
    torch on the CPU, in the reference's execution shape: padded N, query
    chunks, logits materialised in fp32 via ``matmul(k1, (q*k2)^T)``,
    ``masked_fill(finfo.min)``, softmax over the flattened (j,k) pairs, P cast to
    the value dtype, ``P^T @ v1`` then ``(. * v2).sum(k)``.  Follows
    ``src/matterformer/models/simplicial_attention.py``:
      pair mask        :141-145 (pair_key_valid_j & pair_key_valid_k & pair_valid)
      fp32_core        :251-297
      chunk logits     :161-180 (factorized bias :41-47, angle residual :76-81)
      softmax          :317-319
      value path       :326-329, message residual :330-337
      query zeroing    :338-340, final cast :344
    It is the CPU baseline that bench.py times.
    Pinned by: the golden vectors written from the reference itself
    (tests/golden/simplicial_*.npz), ``brute_force_fp64`` below, the closed-form
    KAT of tests/test_simplicial_attention.py:448-463 and the masked-key
    invariance of :415-445 (tests/test_oracle_simplicial.py).

``brute_force_fp64``
    numpy float64, one molecule and head at a time over the valid atoms only:
    S = einsum('d,jd,kd->jk'), softmax over valid pairs, out = einsum('jk,jd,kd->d').
    This is the formula of docs/qm9_edm_matterformer_architecture.md:905-935.
    Also returns lse = logsumexp over the valid pairs
    (triton_simplicial_attention.py:327: lse = m + log l, 0 for empty rows).
    Pinned by: closed forms (q = 0 gives mean_j v1 (.) mean_k v2; a single
    valid pair gives v1_j (.) v2_k; lse of uniform logits is log(#pairs)) and
    agreement with ``reference_path`` in fp32.
"""

from __future__ import annotations

import math

import numpy as np
import torch


def pair_mask(pair_key_valid: torch.Tensor, pair_valid: torch.Tensor | None) -> torch.Tensor:
    """[B,N] key validity (+ optional [B,N,N]) -> [B,N,N] pair validity (simplicial_attention.py:141-145)."""
    pm = pair_key_valid[:, :, None] & pair_key_valid[:, None, :]
    if pair_valid is not None:
        pm = pm & pair_valid.bool()
    return pm


def reference_path(
    q: torch.Tensor,
    k1: torch.Tensor,
    v1: torch.Tensor,
    k2: torch.Tensor,
    v2: torch.Tensor,
    query_valid: torch.Tensor,
    pair_key_valid: torch.Tensor,
    pair_valid: torch.Tensor | None = None,
    *,
    chunk_size: int = 128,
    fp32_core: bool = False,
    factorized_bias: tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
    angle_residual: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
    message_residual: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None,
) -> torch.Tensor:
    """The reference torch path on CPU tensors ``[B,H,N,D]`` (see module docstring)."""
    B, H, N, D = q.shape
    qv = query_valid.bool()
    flat_mask = pair_mask(pair_key_valid.bool(), pair_valid)[:, None, None, :, :].flatten(-2)

    upcast = fp32_core and q.dtype in (torch.float16, torch.bfloat16)
    work = [t.float() if upcast else t for t in (q, k1, v1, k2, v2)]
    qw, k1w, v1w, k2w, v2w = work
    fb = tuple(t.float() for t in factorized_bias) if (factorized_bias is not None and upcast) else factorized_bias
    ar = tuple(t.float() for t in angle_residual) if (angle_residual is not None and upcast) else angle_residual
    mr = tuple(t.float() for t in message_residual) if (message_residual is not None and upcast) else message_residual
    out_dtype = torch.float32 if upcast else v1.dtype
    out = torch.empty(B, H, N, D, dtype=out_dtype)

    for s in range(0, N, chunk_size):
        e = min(N, s + chunk_size)
        qk2 = qw[:, :, s:e, None, :] * k2w[:, :, None, :, :]            # [B,H,c,N,D]
        logits = torch.matmul(k1w[:, :, None, :, :], qk2.transpose(-1, -2)).float()  # [B,H,c,N(j),N(k)]
        if fb is not None:
            u, vb, w, gate = fb
            bias = (u[:, :, s:e, :].float()[..., :, None] + vb[:, :, s:e, :].float()[..., None, :]
                    + w.float()[:, :, None, :, :])
            logits = logits + (gate[:, :, s:e].float()[..., None, None] * bias).to(logits.dtype)
        if ar is not None:
            left, right, agate = ar
            rank = left.shape[-1]
            res = torch.einsum("bhqjr,bhqkr->bhqjk", left[:, :, s:e].float(), right[:, :, s:e].float()) * rank ** -0.5
            logits = logits + (agate[:, :, s:e].float()[..., None, None] * res).to(logits.dtype)
        flat = logits.flatten(-2).masked_fill(~flat_mask, torch.finfo(logits.dtype).min)
        attn = torch.softmax(flat, dim=-1)
        attn = torch.where(flat_mask, attn, torch.zeros_like(attn)).view_as(logits)
        tmp = torch.matmul(attn.to(v1w.dtype).transpose(-2, -1), v1w[:, :, None, :, :])  # [B,H,c,N(k),D]
        chunk_out = (tmp * v2w[:, :, None, :, :]).sum(dim=-2)
        if mr is not None:
            mleft, mright, basis = mr
            rank = mleft.shape[-1]
            coeff = torch.einsum("bhqjk,bhqjr,bhqkr->bhqr", attn.float(), mleft[:, :, s:e].float(),
                                 mright[:, :, s:e].float()) * rank ** -0.5
            chunk_out = chunk_out + torch.einsum("bhqr,hrd->bhqd", coeff, basis.float()).to(chunk_out.dtype)
        chunk_out = chunk_out * qv[:, s:e].to(chunk_out.dtype)[:, None, :, None]
        out[:, :, s:e, :] = chunk_out
    return out.to(v1.dtype)


def brute_force_fp64(
    q: np.ndarray,
    k1: np.ndarray,
    v1: np.ndarray,
    k2: np.ndarray,
    v2: np.ndarray,
    query_valid: np.ndarray,
    pair_key_valid: np.ndarray,
    pair_valid: np.ndarray | None = None,
    *,
    bias: tuple | None = None,
    angle: tuple | None = None,
    message: tuple | None = None,
) -> tuple[np.ndarray, np.ndarray]:
    """float64 reference over valid atoms; returns (out [B,H,N,D], lse [B,H,N]).

    Optional terms (simplicial_attention.py:41-47,76-81,330-337), float64 arrays:
      bias    = (u, v, w, gate): S[j,k] += gate_i (u_ij + v_ik + w_jk)        u,v,w [B,H,N,N], gate [B,H,N]
      angle   = (left, right, gate): S[j,k] += gate_i R^-1/2 sum_r L_ijr R_ikr   [B,H,N,N,R], gate [B,H,N]
      message = (left, right, basis): out_i += sum_r c_r basis[h,r],
                c_r = R^-1/2 sum_jk P_jk L_ijr R_ikr                             basis [H,R,D]
    """
    q, k1, v1, k2, v2 = (np.asarray(a, dtype=np.float64) for a in (q, k1, v1, k2, v2))
    bias = None if bias is None else tuple(np.asarray(a, dtype=np.float64) for a in bias)
    angle = None if angle is None else tuple(np.asarray(a, dtype=np.float64) for a in angle)
    message = None if message is None else tuple(np.asarray(a, dtype=np.float64) for a in message)
    B, H, N, D = q.shape
    out = np.zeros((B, H, N, D))
    lse = np.zeros((B, H, N))
    for b in range(B):
        keys = np.flatnonzero(pair_key_valid[b])
        queries = np.flatnonzero(query_valid[b])
        if keys.size == 0 or queries.size == 0:
            continue
        pm = np.ones((keys.size, keys.size), dtype=bool)
        if pair_valid is not None:
            pm = pair_valid[b][np.ix_(keys, keys)].astype(bool)
        if not pm.any():
            continue
        for h in range(H):
            K1, V1, K2, V2 = k1[b, h, keys], v1[b, h, keys], k2[b, h, keys], v2[b, h, keys]
            for i in queries:
                S = np.einsum("d,jd,kd->jk", q[b, h, i], K1, K2)
                if bias is not None:
                    u, v, w, gate = bias
                    S = S + gate[b, h, i] * (u[b, h, i, keys][:, None] + v[b, h, i, keys][None, :]
                                             + w[b, h][np.ix_(keys, keys)])
                if angle is not None:
                    left, right, gate = angle
                    L, R = left[b, h, i, keys], right[b, h, i, keys]
                    S = S + gate[b, h, i] * (L @ R.T) / math.sqrt(L.shape[-1])
                S = np.where(pm, S, -np.inf)
                m = S.max()
                P = np.exp(S - m)
                tot = P.sum()
                P /= tot
                out[b, h, i] = np.einsum("jk,jd,kd->d", P, V1, V2)
                if message is not None:
                    left, right, basis = message
                    L, R = left[b, h, i, keys], right[b, h, i, keys]
                    c = np.einsum("jk,jr,kr->r", P, L, R) / math.sqrt(L.shape[-1])
                    out[b, h, i] += c @ basis[h]
                lse[b, h, i] = m + math.log(tot)
    return out, lse


def work_flops(pair_key_valid: np.ndarray, query_valid: np.ndarray, heads: int, head_dim: int) -> int:
    """Algorithmic FLOPs of the valid work: sum_b 4*H*D*n_q(b)*n_k(b)^2."""
    nk = np.asarray(pair_key_valid).astype(bool).sum(axis=1).astype(np.int64)
    nq = np.asarray(query_valid).astype(bool).sum(axis=1).astype(np.int64)
    return int(4 * heads * head_dim * np.sum(nq * nk * nk))
