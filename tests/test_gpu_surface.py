"""GPU tests of the drop-in Python surface and of kernel paths the shape tests do not reach.

Counterparts of the reference's GPU tests (tests/test_simplicial_attention.py:817-1020 of
stases/Matterformer), run against this package's HIP backend:

  :819-824   explicit "triton" rejects float64 with the reference's message
  :829-836   eval-mode dropout still takes the fused path
  :841-896   no-bias forward + backward through the 21-argument Function, 1e-4
  :901-1020  factorized + angle + message forward + backward, 1e-4

plus: SimplicialAttention dispatch for impl in {auto, torch, triton, hip}; tf32
(served by the fp32 MFMA path, so bit-identical to ieee_fp32); the 16-bit
kernel for more than 512 tokens and for outputs that are not 16-byte aligned
(simplicial_fast.hip) and for operands that are not (the general kernel);
config 2 molecule by molecule with a per-row bound; every lane-count variant
of the kNN kernel bit-exact; two graphs captured on one stream.
"""

import ctypes
import math

import numpy as np
import pytest
import torch

from matterformer_amd import _native
from matterformer_amd.geometry_ops import knn_graph
from matterformer_amd.hip_simplicial_attention import hip_simplicial_attention_forward
from matterformer_amd.simplicial_attention import (
    SimplicialAttention,
    SimplicialAttentionMask,
    SimplicialFactorizedBias,
    SimplicialLowRankAngleResidual,
    SimplicialLowRankMessageResidual,
    TwoSimplicialAttention,
    _TritonTwoSimplicialAttentionFunction,
    simplicial_attention_torch_from_projected,
)
from matterformer_amd.workloads import random_simplicial, simplicial_workload
from oracle.native import knn as oracle_knn
from oracle.simplicial import brute_force_fp64

pytestmark = pytest.mark.gpu


def rel_err(got, ref):
    got = np.asarray(got, dtype=np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


def apply_function(q, k1, v1, k2, v2, mask, *, fb=None, ar=None, mr=None, basis=None, precision="ieee_fp32",
                   chunk_size=2, debug=False):
    """The reference tests' _apply_triton_function (tests/test_simplicial_attention.py:187-241)."""
    empty = q.new_empty(0)
    pv = mask.pair_valid if mask.pair_valid is not None else torch.empty(0, device=q.device, dtype=torch.bool)
    u, v, w, gate = (fb.u, fb.v, fb.w, fb.gate) if fb is not None else (empty,) * 4
    al, arr, ag = (ar.left, ar.right, ar.gate) if ar is not None else (empty,) * 3
    ml, mrr, mb = (mr.left, mr.right, basis) if mr is not None else (empty,) * 3
    return _TritonTwoSimplicialAttentionFunction.apply(
        q, k1, v1, k2, v2, mask.query_valid, mask.pair_key_valid, pv, u, v, w, gate, al, arr, ag, ml, mrr, mb,
        precision, chunk_size, debug)


# ---------------------------------------------------------------------- module surface

def test_explicit_triton_rejects_unsupported_dtype(cuda):
    attn = TwoSimplicialAttention(dim=32, num_heads=4, impl="triton").to(device=cuda, dtype=torch.float32)
    x = torch.randn(2, 4, 32, device=cuda, dtype=torch.float64)
    with pytest.raises(RuntimeError, match="only supports float16/bfloat16/float32"):
        attn(x)


def test_eval_mode_dropout_allows_fused_path(cuda):
    torch.manual_seed(0)
    attn = TwoSimplicialAttention(dim=32, num_heads=4, impl="auto", dropout=0.1, precision="ieee_fp32").to(cuda)
    attn.eval()
    attn(torch.randn(2, 5, 32, device=cuda))
    assert attn._last_impl_used == "triton"
    attn.train()
    attn(torch.randn(2, 5, 32, device=cuda))
    assert attn._last_impl_used == "torch"


@pytest.mark.parametrize("impl", ["auto", "torch", "triton", "hip"])
def test_module_dispatch_and_outputs(cuda, impl):
    torch.manual_seed(1)
    attn = SimplicialAttention(dim=64, num_heads=4, impl=impl, precision="ieee_fp32").to(cuda)
    x = torch.randn(3, 11, 64, device=cuda)
    kpm = torch.zeros(3, 11, dtype=torch.bool, device=cuda)
    kpm[1, 7:] = True
    kpm[2, 2:] = True
    out = attn(x, key_padding_mask=kpm)
    assert attn._last_impl_used == ("torch" if impl == "torch" else "triton")
    q, k1, v1, k2, v2 = attn._project_inputs(x)
    mask = SimplicialAttentionMask.from_key_padding_mask(kpm, batch_size=3, num_tokens=11, device=cuda)
    heads = simplicial_attention_torch_from_projected(q, k1, v1, k2, v2, attention_mask=mask, fp32_core=True)
    torch.testing.assert_close(out, attn.out_proj(attn._merge_heads(heads)), rtol=1e-4, atol=1e-4)


def test_module_bf16_precision_matches_fp32_torch_path(cuda):
    torch.manual_seed(2)
    attn = SimplicialAttention(dim=128, num_heads=2, impl="auto", precision="bf16_tc").to(cuda)
    x = torch.randn(4, 23, 128, device=cuda)
    kpm = torch.arange(23, device=cuda)[None, :] >= torch.tensor([23, 19, 9, 1], device=cuda)[:, None]
    out = attn(x, key_padding_mask=kpm)
    assert attn._last_impl_used == "triton" and out.dtype == torch.float32
    attn.impl = "torch"
    ref = attn(x, key_padding_mask=kpm)
    assert rel_err(out.detach().cpu(), ref.detach().cpu().double().numpy()) <= 2e-2


# ---------------------------------------------------------------- Function + backward

def _leaves(shape, device, seed, scale=1.0):
    gen = torch.Generator().manual_seed(seed)
    base = [torch.randn(shape, generator=gen) * scale for _ in range(5)]
    return [t.to(device).requires_grad_(True) for t in base]


def test_no_bias_forward_backward_matches_torch_path(cuda):
    """Reference test :841-896: fp32 core torch path vs the Function, forward and gradients at 1e-4."""
    ref = _leaves((2, 4, 5, 8), cuda, seed=0)
    got = [t.detach().clone().requires_grad_(True) for t in ref]
    kpm = torch.tensor([[False, False, False, False, True], [False, False, True, True, True]], device=cuda)
    mask = SimplicialAttentionMask.from_key_padding_mask(kpm, batch_size=2, num_tokens=5, device=cuda)
    expected = simplicial_attention_torch_from_projected(*ref, attention_mask=mask, chunk_size=2, fp32_core=True)
    out = apply_function(*got, mask)
    torch.testing.assert_close(out, expected, rtol=1e-4, atol=1e-4)
    expected.square().mean().backward()
    out.square().mean().backward()
    for a, e in zip(got, ref):
        torch.testing.assert_close(a.grad, e.grad, rtol=1e-4, atol=1e-4)


def test_all_terms_forward_backward_matches_torch_path(cuda):
    """Reference test :901-1020: factorized bias, angle and message, forward and every gradient at 1e-4."""
    torch.manual_seed(0)
    B, H, N, D = 1, 2, 7, 8
    ref = _leaves((B, H, N, D), cuda, seed=3)
    got = [t.detach().clone().requires_grad_(True) for t in ref]

    def pair(*shape):
        return torch.randn(*shape, device=cuda).requires_grad_(True)

    fb_ref = SimplicialFactorizedBias(pair(B, H, N, N), pair(B, H, N, N), pair(B, H, N, N), pair(B, H, N))
    ar_ref = SimplicialLowRankAngleResidual(pair(B, H, N, N, 5), pair(B, H, N, N, 5), pair(B, H, N))
    mr_ref = SimplicialLowRankMessageResidual(pair(B, H, N, N, 3), pair(B, H, N, N, 3))
    basis_ref = pair(H, 3, D)

    def clone(t):
        return t.detach().clone().requires_grad_(True)

    fb = SimplicialFactorizedBias(*(clone(t) for t in (fb_ref.u, fb_ref.v, fb_ref.w, fb_ref.gate)))
    ar = SimplicialLowRankAngleResidual(*(clone(t) for t in (ar_ref.left, ar_ref.right, ar_ref.gate)))
    mr = SimplicialLowRankMessageResidual(clone(mr_ref.left), clone(mr_ref.right))
    basis = clone(basis_ref)
    kpm = torch.tensor([[False] * 5 + [True] * 2], device=cuda)
    pv = torch.ones(B, N, N, dtype=torch.bool, device=cuda)
    pv[:, 1, 4] = False
    pv[:, 4, 1] = False
    base = SimplicialAttentionMask.from_key_padding_mask(kpm, batch_size=B, num_tokens=N, device=cuda)
    mask = SimplicialAttentionMask(query_valid=base.query_valid, pair_key_valid=base.pair_key_valid, pair_valid=pv)
    expected = simplicial_attention_torch_from_projected(
        *ref, attention_mask=mask, factorized_bias=fb_ref, angle_residual=ar_ref, message_residual=mr_ref,
        message_basis=basis_ref, chunk_size=3, fp32_core=True)
    out = apply_function(*got, mask, fb=fb, ar=ar, mr=mr, basis=basis, chunk_size=3)
    torch.testing.assert_close(out, expected, rtol=1e-4, atol=1e-4)
    expected.square().mean().backward()
    out.square().mean().backward()
    pairs = list(zip(got, ref)) + [
        (fb.u, fb_ref.u), (fb.v, fb_ref.v), (fb.w, fb_ref.w), (fb.gate, fb_ref.gate),
        (ar.left, ar_ref.left), (ar.right, ar_ref.right), (ar.gate, ar_ref.gate),
        (mr.left, mr_ref.left), (mr.right, mr_ref.right), (basis, basis_ref)]
    for a, e in pairs:
        torch.testing.assert_close(a.grad, e.grad, rtol=1e-4, atol=1e-4)


def test_function_backward_matches_fp64_autograd(cuda):
    """Gradients of the Function against float64 autograd on the CPU (B=3, ragged, pair mask)."""
    B, H, N, D = 3, 2, 19, 32
    case = random_simplicial(B, H, N, D, seed=41, counts=[19, 11, 4], holes=[(0, 2)], pair_drop=0.15,
                            std=(4.0 / D) ** (1 / 6))
    q, k1, v1, k2, v2, qv, pkv, pv = case
    mask_cpu = SimplicialAttentionMask(query_valid=qv, pair_key_valid=pkv, pair_valid=pv)
    ref = [t.double().requires_grad_(True) for t in (q, k1, v1, k2, v2)]
    expected = simplicial_attention_torch_from_projected(*ref, attention_mask=mask_cpu, chunk_size=8)
    gen = torch.Generator().manual_seed(5)
    go = torch.randn(B, H, N, D, generator=gen)
    (expected * go.double()).sum().backward()
    got = [t.to(cuda).requires_grad_(True) for t in (q, k1, v1, k2, v2)]
    mask = SimplicialAttentionMask(query_valid=qv.to(cuda), pair_key_valid=pkv.to(cuda), pair_valid=pv.to(cuda))
    out = apply_function(*got, mask)
    (out * go.to(cuda)).sum().backward()
    np.testing.assert_allclose(out.detach().cpu().numpy(), expected.detach().numpy(), rtol=1e-4, atol=1e-4)
    for a, e in zip(got, ref):
        np.testing.assert_allclose(a.grad.cpu().numpy(), e.grad.numpy(), rtol=1e-4, atol=1e-4)


# ------------------------------------------------------------------ precision modes

def test_tf32_runs_the_fp32_path(cuda):
    case = random_simplicial(2, 2, 33, 32, seed=17, counts=[33, 20], std=(4.0 / 32) ** (1 / 6))
    q, k1, v1, k2, v2, qv, pkv, pv = case
    ops = [t.to(cuda) for t in (q, k1, v1, k2, v2)]
    kw = dict(query_valid=qv.to(cuda), pair_key_valid=pkv.to(cuda), pair_valid=None)
    tf32 = hip_simplicial_attention_forward(*ops, precision="tf32", **kw)
    ieee = hip_simplicial_attention_forward(*ops, precision="ieee_fp32", **kw)
    torch.cuda.synchronize()
    ref, ref_lse = brute_force_fp64(*(t.double().numpy() for t in (q, k1, v1, k2, v2)), qv.numpy(), pkv.numpy())
    np.testing.assert_allclose(tf32[2].cpu().numpy(), ref, rtol=1e-4, atol=1e-4)
    assert torch.equal(tf32[2], ieee[2]) and torch.equal(tf32[1], ieee[1])
    b16 = [t.to(torch.bfloat16) for t in ops]
    tf32_b16 = hip_simplicial_attention_forward(*b16, precision="tf32", **kw)
    ieee_b16 = hip_simplicial_attention_forward(*b16, precision="ieee_fp32", **kw)
    assert tf32_b16[0].dtype == torch.bfloat16 and torch.equal(tf32_b16[2], ieee_b16[2])


# ------------------------------------------------------------- simplicial_fast.hip

def _oracle_rows(case, dtype, rows):
    """float64 brute force on selected query rows only (other rows come back 0)."""
    q, k1, v1, k2, v2, qv, pkv, pv = case
    sel = torch.zeros_like(qv)
    for b, idx in rows.items():
        sel[b, idx] = qv[b, idx]
    return brute_force_fp64(*(t.to(dtype).double().numpy() for t in (q, k1, v1, k2, v2)), sel.numpy(),
                            pkv.numpy(), None if pv is None else pv.numpy()), sel


@pytest.mark.parametrize("std", [0.05, 0.6], ids=["bound", "twopass"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_more_than_512_tokens(cuda, dtype, std):
    """N = 600 (beyond the pair kernel) runs simplicial_fast.hip; holes and pair_valid, sampled rows.

    std 0.05 keeps every query's logit bound below the direct-exp limit; std 0.6 puts it near 250,
    past the limit (60 for bf16, 14 for fp16), so every query takes the exact-maximum two-pass mode,
    while the logits keep a standard deviation near 1.7.  (At std 1.3 the logits reach |S| ~ 80 and the
    bf16 rounding of the q (.) k1 products alone -- the reference kernel rounds q (.) k2 the same way --
    moves the softmax by about 2 %.)"""
    B, H, N, D = 2, 2, 600, 64
    case = random_simplicial(B, H, N, D, seed=600 + int(std * 10), counts=[600, 531], holes=[(0, 17), (1, 300)],
                            pair_drop=0.1, std=std)
    q, k1, v1, k2, v2, qv, pkv, pv = case
    out, lse, out32 = hip_simplicial_attention_forward(
        *(t.to(dtype).to(cuda) for t in (q, k1, v1, k2, v2)), query_valid=qv.to(cuda), pair_key_valid=pkv.to(cuda),
        pair_valid=pv.to(cuda), precision="bf16_tc")
    torch.cuda.synchronize()
    gen = torch.Generator().manual_seed(9)
    rows = {b: torch.randperm(int(qv[b].sum()), generator=gen)[:12] for b in range(B)}
    (ref, ref_lse), sel = _oracle_rows(case, dtype, rows)
    m = sel[:, None, :].expand(B, H, N).numpy()
    got = out32.cpu().numpy()
    assert rel_err(got[m], ref[m]) <= 2e-2
    np.testing.assert_allclose(lse.cpu().numpy()[m], ref_lse[m], rtol=2e-2, atol=5e-2)
    assert torch.count_nonzero(out32.cpu().permute(0, 2, 1, 3)[~qv]) == 0


def _capi_call(ops, qv, pkv, dtype, out, out_f32, lse):
    B, H, N, D = ops[0].shape
    lib = _native.lib()
    code = _native.dtype_code(dtype)
    nbytes = lib.mf_simplicial_fwd_workspace_size(B, H, N, D, code)
    ws = torch.zeros(int(nbytes), dtype=torch.uint8, device=ops[0].device)
    args = _native.MfSimplicialFwdArgs(
        q=ops[0].data_ptr(), k1=ops[1].data_ptr(), v1=ops[2].data_ptr(), k2=ops[3].data_ptr(), v2=ops[4].data_ptr(),
        query_valid=qv.data_ptr(), pair_key_valid=pkv.data_ptr(), pair_valid=None,
        out=None if out is None else out.data_ptr(), out_f32=None if out_f32 is None else out_f32.data_ptr(),
        lse=None if lse is None else lse.data_ptr(), workspace=ws.data_ptr(), workspace_bytes=nbytes,
        batch=B, heads=H, tokens=N, head_dim=D, dtype=code, precision=0)
    _native.check(lib.mf_simplicial_fwd(ctypes.byref(args), _native.current_stream(ops[0].device)), "mf_simplicial_fwd")
    torch.cuda.synchronize()
    return ws


def _offset_view(shape, dtype, device, offset_elems):
    n = math.prod(shape)
    flat = torch.zeros(n + 16, dtype=dtype, device=device)
    return flat[offset_elems:offset_elems + n].view(shape)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_capi_unaligned_outputs_run_fast_kernel(cuda, dtype):
    """Outputs 8 bytes off a 16-byte boundary (operands aligned) take simplicial_fast.hip."""
    B, H, N, D = 3, 2, 45, 64
    case = random_simplicial(B, H, N, D, seed=45, counts=[45, 30, 7], holes=[(1, 3)], std=0.3)
    q, k1, v1, k2, v2, qv, pkv, _ = case
    ops = [t.to(dtype).to(cuda).contiguous() for t in (q, k1, v1, k2, v2)]
    out = _offset_view((B, H, N, D), dtype, cuda, 4)     # 8 bytes off
    out32 = _offset_view((B, H, N, D), torch.float32, cuda, 2)
    lse = _offset_view((B, H, N), torch.float32, cuda, 1)
    assert out.data_ptr() % 16 == 8 and out32.data_ptr() % 16 == 8
    _capi_call(ops, qv.to(torch.uint8).to(cuda), pkv.to(torch.uint8).to(cuda), dtype, out, out32, lse)
    ref, ref_lse = brute_force_fp64(*(t.to(dtype).double().numpy() for t in (q, k1, v1, k2, v2)), qv.numpy(),
                                    pkv.numpy())
    assert rel_err(out32.cpu().numpy(), ref) <= 2e-2
    assert rel_err(out.float().cpu().numpy(), ref) <= 2e-2
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=2e-2, atol=5e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_capi_unaligned_operands_run_general_kernel(cuda, dtype):
    """Operands 2 bytes off a 16-byte boundary take the general kernel's element-wise staging."""
    B, H, N, D = 2, 2, 37, 64
    case = random_simplicial(B, H, N, D, seed=37, counts=[37, 12], std=0.3)
    q, k1, v1, k2, v2, qv, pkv, _ = case
    ops = []
    for t in (q, k1, v1, k2, v2):
        view = _offset_view((B, H, N, D), dtype, cuda, 1)
        view.copy_(t.to(dtype))
        ops.append(view)
    assert ops[0].data_ptr() % 16 == 2
    out = torch.empty(B, H, N, D, dtype=dtype, device=cuda)
    out32 = torch.empty(B, H, N, D, dtype=torch.float32, device=cuda)
    _capi_call(ops, qv.to(torch.uint8).to(cuda), pkv.to(torch.uint8).to(cuda), dtype, out, out32, None)
    ref, _ = brute_force_fp64(*(t.to(dtype).double().numpy() for t in (q, k1, v1, k2, v2)), qv.numpy(), pkv.numpy())
    assert rel_err(out32.cpu().numpy(), ref) <= 2e-2


# ------------------------------------------------------------ config 2, every molecule

def test_geom_config_every_molecule_per_row(cuda):
    """Config 2 at full size: all 64 molecules against float64, normwise and row by row."""
    w = simplicial_workload("geom")
    wd = w.to(cuda, torch.bfloat16)
    out, lse, out32 = hip_simplicial_attention_forward(
        wd.q, wd.k1, wd.v1, wd.k2, wd.v2, query_valid=wd.query_valid, pair_key_valid=wd.pair_key_valid,
        pair_valid=None, precision="bf16_tc")
    torch.cuda.synchronize()
    ref, ref_lse = brute_force_fp64(*(t.to(torch.bfloat16).double().numpy() for t in (w.q, w.k1, w.v1, w.k2, w.v2)),
                                    w.query_valid.numpy(), w.pair_key_valid.numpy())
    got = out32.cpu().numpy()
    assert rel_err(got, ref) <= 2e-2
    rows = w.query_valid[:, None, :].expand(-1, w.shape[1], -1).numpy()
    diff = np.linalg.norm(got - ref, axis=-1)[rows]
    norm = np.linalg.norm(ref, axis=-1)[rows]
    print(f"config 2: worst row {(diff / norm).max():.3e}, median {np.median(diff / norm):.3e}", flush=True)
    # measured worst row 6.2e-4 (median 3.1e-4): the bar is five times the worst
    assert (diff / norm).max() <= 3e-3, (diff / norm).max()
    for b in range(w.shape[0]):
        assert rel_err(got[b], ref[b]) <= 2e-2, b
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=2e-2, atol=5e-2)


# ---------------------------------------------------------------- kNN lane variants

@pytest.mark.parametrize("B,k", [(200, 16), (400, 16), (800, 8), (1500, 16)],
                         ids=["L8", "L4", "L2", "L1"])
def test_knn_every_lane_count_bitwise(cuda, B, k):
    """Batch sizes that select 8, 4, 2 and 1 lanes per query on 256 CUs (k <= 16 kernels), bit-exact."""
    N = 181
    gen = torch.Generator().manual_seed(B + k)
    coords = torch.randn(B, N, 3, generator=gen) * math.sqrt(2.0)
    pad = torch.rand(B, N, generator=gen) < 0.05
    print(f"knn lanes B={B} N={N} k={k}", flush=True)
    idx, dist = knn_graph(coords.to(cuda), k, pad.to(cuda))
    torch.cuda.synchronize()
    ridx, rdist = oracle_knn(coords.numpy(), k, pad.numpy())
    assert np.array_equal(idx.cpu().numpy(), ridx)
    assert np.array_equal(dist.cpu().numpy().view(np.uint32), rdist.view(np.uint32))


# ------------------------------------------------------------------- graph capture

def test_two_graphs_on_one_stream_have_their_own_workspace(cuda):
    B, H, N, D = 5, 2, 33, 64
    q, k1, v1, k2, v2, qv, pkv, _ = random_simplicial(B, H, N, D, seed=77, counts=[33, 20, 9, 31, 2], std=0.1)
    ops = [t.to(torch.bfloat16).to(cuda) for t in (q, k1, v1, k2, v2)]
    masks = dict(query_valid=qv.to(cuda), pair_key_valid=pkv.to(cuda), pair_valid=None, precision="bf16_tc")
    eager = hip_simplicial_attention_forward(*ops, **masks)[2].clone()
    side = torch.cuda.Stream(cuda)
    side.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(side):
        hip_simplicial_attention_forward(*ops, **masks)
    torch.cuda.current_stream(cuda).wait_stream(side)
    torch.cuda.synchronize()
    before = len(_native._CAPTURED_WORKSPACES)
    graphs, outs = [], []
    for _ in range(2):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            outs.append(hip_simplicial_attention_forward(*ops, **masks)[2])
        graphs.append(g)
    captured = _native._CAPTURED_WORKSPACES[before:]
    assert len(captured) == 2 and captured[0].data_ptr() != captured[1].data_ptr()
    for rep in range(3):
        for g, o in zip(graphs, outs):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(o, eager), rep
        again = hip_simplicial_attention_forward(*ops, **masks)[2]
        torch.cuda.synchronize()
        assert torch.equal(again, eager), rep
