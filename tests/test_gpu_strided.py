"""GPU tests of the ABI 8 operand strides of mf_simplicial_fwd.

The module path (simplicial_attention.py:695-733,897-987 of stases/Matterformer)
splits one in_proj output into five [B, H, N, D] head views and copies each with
.contiguous() (_split_heads, :708-711), and merges the output heads with another
copy (_merge_heads).  Here the pair kernel reads the views in place through
their {batch, head, token} strides and writes the merged [B, N, H, D] layout.
The kernel does the same arithmetic on the same values either way, so every
check against the contiguous call is bitwise; the module output is also checked
against the float64 brute force of oracle/simplicial.py (2e-2 normwise, the
16-bit bar of the other GPU tests) and its gradients against the contiguous
route's.
"""

import ctypes

import numpy as np
import pytest
import torch

from matterformer_amd import _native
from matterformer_amd.hip_simplicial_attention import hip_simplicial_attention_forward
from matterformer_amd.simplicial_attention import SimplicialAttention
from matterformer_amd.simplicial_types import SimplicialAttentionMask
from matterformer_amd.workloads import random_simplicial
from oracle.simplicial import brute_force_fp64

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _views(B, H, N, D, dtype, seed):
    """Five [B, H, N, D] views of one [B, N, 5 * H * D] projection output, q rescaled as the module does
    (a new tensor in the projection's token-major order) and k1, v1, k2, v2 left as chunk views."""
    gen = torch.Generator().manual_seed(seed)
    proj = (torch.randn(B, N, 5 * H * D, generator=gen) * 0.2).to(DEV, dtype)
    parts = [p.view(B, N, H, D).transpose(1, 2) for p in proj.chunk(5, dim=-1)]
    parts[0] = parts[0] * (D ** -0.5)
    return parts


def _masks(B, N, seed, holes=False):
    gen = torch.Generator().manual_seed(seed)
    counts = torch.randint(max(1, N // 3), N + 1, (B,), generator=gen)
    valid = torch.arange(N)[None, :] < counts[:, None]
    if holes:
        valid[:, 1] = False
    return valid.to(DEV), valid.clone().to(DEV)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,H,N,D", [(5, 4, 37, 64), (3, 2, 90, 32), (2, 8, 181, 64)])
@pytest.mark.parametrize("holes", [False, True])
def test_views_match_contiguous_bitwise(dtype, B, H, N, D, holes):
    q, k1, v1, k2, v2 = _views(B, H, N, D, dtype, seed=B * 100 + N)
    assert not k1.is_contiguous() and not q.is_contiguous()
    qv, pkv = _masks(B, N, seed=N, holes=holes)
    prec = "bf16_tc"
    out_v, lse_v, o32_v = hip_simplicial_attention_forward(q, k1, v1, k2, v2, query_valid=qv, pair_key_valid=pkv,
                                                           pair_valid=None, precision=prec)
    ref = [t.contiguous() for t in (q, k1, v1, k2, v2)]
    out_c, lse_c, o32_c = hip_simplicial_attention_forward(*ref, query_valid=qv, pair_key_valid=pkv,
                                                           pair_valid=None, precision=prec)
    torch.cuda.synchronize()
    # the views path writes the merged [B, N, H, D] layout
    assert out_v.shape == (B, H, N, D) and out_v.permute(0, 2, 1, 3).is_contiguous()
    assert torch.equal(out_v, out_c)
    assert torch.equal(o32_v, o32_c)
    assert torch.equal(lse_v, lse_c)


def test_views_with_factorized_bias_match_contiguous_bitwise():
    B, H, N, D = 3, 4, 45, 64
    q, k1, v1, k2, v2 = _views(B, H, N, D, torch.bfloat16, seed=7)
    qv, pkv = _masks(B, N, seed=3)
    gen = torch.Generator().manual_seed(11)
    bias = [(torch.randn(B, H, N, N, generator=gen) * 0.5).to(DEV, torch.bfloat16) for _ in range(3)]
    gate = torch.randn(B, H, N, generator=gen).to(DEV, torch.bfloat16)
    kw = dict(query_valid=qv, pair_key_valid=pkv, pair_valid=None, u=bias[0], v_bias=bias[1], w=bias[2],
              gate=gate, precision="bf16_tc")
    out_v, lse_v, _ = hip_simplicial_attention_forward(q, k1, v1, k2, v2, **kw)
    out_c, lse_c, _ = hip_simplicial_attention_forward(*(t.contiguous() for t in (q, k1, v1, k2, v2)), **kw)
    torch.cuda.synchronize()
    assert torch.equal(out_v, out_c)
    assert torch.equal(lse_v, lse_c)


def _capi_args(q, kv_stride, out, dtype_code, q_stride=(0, 0, 0), out_stride=(0, 0, 0)):
    B, H, N, D = q.shape
    valid = torch.ones(B, N, dtype=torch.bool, device=DEV)
    lib = _native.lib()
    ws_bytes = lib.mf_simplicial_fwd_workspace_size(B, H, N, D, dtype_code)
    ws = _native.workspace(ws_bytes, DEV)
    keep = [valid, ws]
    args = _native.MfSimplicialFwdArgs(
        q=q.data_ptr(), k1=q.data_ptr(), v1=q.data_ptr(), k2=q.data_ptr(), v2=q.data_ptr(),
        query_valid=valid.data_ptr(), pair_key_valid=valid.data_ptr(), pair_valid=None,
        out=out.data_ptr(), out_f32=None, lse=None,
        workspace=None if ws is None else ws.data_ptr(), workspace_bytes=ws_bytes,
        batch=B, heads=H, tokens=N, head_dim=D, dtype=dtype_code, precision=_native.MF_PREC["bf16_tc"],
        q_stride=(ctypes.c_int64 * 3)(*q_stride), kv_stride=(ctypes.c_int64 * 3)(*kv_stride),
        out_stride=(ctypes.c_int64 * 3)(*out_stride))
    return lib, args, keep


def test_capi_rejects_strides_off_the_pair_kernel():
    """fp32 operands never run the pair kernel: non-default strides are refused before any launch."""
    B, H, N, D = 2, 2, 16, 32
    q = torch.randn(B, H, N, D, device=DEV)
    out = torch.empty_like(q)
    lib, args, keep = _capi_args(q, (H * N * D, N * D, D + 8), out, _native.MF_DTYPE_F32)
    status = lib.mf_simplicial_fwd(args, _native.current_stream(DEV))
    assert status == _native.MF_ERR_UNSUPPORTED
    assert b"pair kernel only" in lib.mf_last_error()


def test_capi_rejects_strides_not_multiple_of_8():
    B, H, N, D = 2, 2, 16, 32
    q = torch.randn(B, H, N, D, device=DEV).to(torch.bfloat16)
    out = torch.empty_like(q)
    lib, args, keep = _capi_args(q, (H * N * D, N * D, D + 4), out, _native.MF_DTYPE_BF16)
    status = lib.mf_simplicial_fwd(args, _native.current_stream(DEV))
    assert status == _native.MF_ERR_INVALID_ARGUMENT
    assert b"multiples of 8" in lib.mf_last_error()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_module_views_path_forward_and_gradients(dtype):
    """SimplicialAttention(impl="hip") on padded molecules: the output against float64, and forward and
    gradients bitwise against the same module routed through contiguous copies."""
    B, N, dim, H = 4, 53, 256, 4
    D = dim // H
    torch.manual_seed(5)
    attn = SimplicialAttention(dim, H, impl="hip", precision="bf16_tc").to(DEV, dtype)
    gen = torch.Generator().manual_seed(6)
    x0 = torch.randn(B, N, dim, generator=gen).to(DEV, dtype)
    qv, pkv = _masks(B, N, seed=9)
    pad = ~pkv
    mask = SimplicialAttentionMask.from_key_padding_mask(pad, batch_size=B, num_tokens=N, device=DEV)

    x = x0.clone().requires_grad_(True)
    out = attn(x, attention_mask=mask)
    out.float().square().mean().backward()
    grads = [x.grad.clone()] + [p.grad.clone() for p in attn.parameters()]
    attn.zero_grad(set_to_none=True)

    # the same module with the projections copied before the call (the contiguous layout)
    orig = attn._forward_triton

    def contiguous_route(q, k1, v1, k2, v2, **kw):
        return orig(*(t.contiguous() for t in (q, k1, v1, k2, v2)), **kw)

    attn._forward_triton = contiguous_route
    try:
        x2 = x0.clone().requires_grad_(True)
        out2 = attn(x2, attention_mask=mask)
        out2.float().square().mean().backward()
    finally:
        attn._forward_triton = orig
    grads2 = [x2.grad] + [p.grad for p in attn.parameters()]
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    for g1, g2 in zip(grads, grads2):
        assert torch.equal(g1, g2)

    # the attention output of the views path against float64 on the same 16-bit projections
    with torch.no_grad():
        q, k1, v1, k2, v2 = attn._project_inputs(x0)
        o, _, _ = hip_simplicial_attention_forward(q, k1, v1, k2, v2, query_valid=qv, pair_key_valid=pkv,
                                                   pair_valid=None, precision="bf16_tc", need_backward_state=False)
    ref, _ = brute_force_fp64(*(t.double().cpu().numpy() for t in (q, k1, v1, k2, v2)), qv.cpu().numpy(),
                              pkv.cpu().numpy())
    got = o.double().cpu().numpy()
    err = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
    assert err <= 2e-2, err


def test_bias_batch_slices_read_their_own_molecules():
    """More molecules than one pair-kernel launch takes (256): the second slice's factorized bias comes
    from its own molecules.  Checked on molecules of both slices against float64."""
    B, H, N, D = 260, 1, 12, 32
    q, k1, v1, k2, v2, qv, pkv, _ = random_simplicial(B, H, N, D, seed=21, std=0.5)
    gen = torch.Generator().manual_seed(22)
    bias = [torch.randn(B, H, N, N, generator=gen) * 0.5 for _ in range(3)] + [torch.randn(B, H, N, generator=gen)]
    ops = [t.to(DEV, torch.bfloat16) for t in (q, k1, v1, k2, v2)]
    bs = [t.to(DEV, torch.bfloat16) for t in bias]
    _, _, o32 = hip_simplicial_attention_forward(*ops, query_valid=qv.to(DEV), pair_key_valid=pkv.to(DEV),
                                                 pair_valid=None, u=bs[0], v_bias=bs[1], w=bs[2], gate=bs[3],
                                                 precision="bf16_tc")
    torch.cuda.synchronize()
    pick = [0, 1, 255, 256, 258, 259]
    sel = lambda t: t[pick].double().cpu().numpy()  # noqa: E731
    ref, _ = brute_force_fp64(*(sel(t) for t in ops), qv[pick].numpy(), pkv[pick].numpy(),
                              bias=tuple(sel(t) for t in bs))
    got = o32[pick].double().cpu().numpy()
    for n, b in enumerate(pick):
        err = float(np.linalg.norm(got[n] - ref[n]) / max(np.linalg.norm(ref[n]), 1e-30))
        assert err <= 2e-2, (b, err)


def test_views_with_pair_valid_fall_back_to_copies():
    """Strided operands are not taken together with pair_valid: the launcher copies the views instead, and
    a direct C-ABI call with both is refused."""
    B, H, N, D = 2, 4, 33, 64
    q, k1, v1, k2, v2 = _views(B, H, N, D, torch.bfloat16, seed=17)
    qv, pkv = _masks(B, N, seed=4)
    gen = torch.Generator().manual_seed(18)
    pv = (torch.rand(B, N, N, generator=gen) > 0.3).to(DEV)
    kw = dict(query_valid=qv, pair_key_valid=pkv, pair_valid=pv, precision="bf16_tc")
    out_v, lse_v, _ = hip_simplicial_attention_forward(q, k1, v1, k2, v2, **kw)
    out_c, lse_c, _ = hip_simplicial_attention_forward(*(t.contiguous() for t in (q, k1, v1, k2, v2)), **kw)
    torch.cuda.synchronize()
    assert out_v.is_contiguous()  # the copies' contiguous output layout
    assert torch.equal(out_v, out_c) and torch.equal(lse_v, lse_c)

    qc = q.contiguous()
    out = torch.empty_like(qc)
    lib, args, keep = _capi_args(qc, (H * N * D, N * D, D), out, _native.MF_DTYPE_BF16)
    args.pair_valid = pv.data_ptr()
    status = lib.mf_simplicial_fwd(args, _native.current_stream(DEV))
    assert status == _native.MF_ERR_UNSUPPORTED
    assert b"no pair_valid" in lib.mf_last_error()
