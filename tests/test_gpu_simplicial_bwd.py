"""GPU parity of the deterministic HIP backward (mf_simplicial_bwd) against float64 autograd.

The checker is autograd of the product's torch path (matterformer_amd.simplicial_types,
bit-identical to the reference's torch path on every committed fixture) run in
float64 on the CPU over the same inputs, i.e. the gradient of
simplicial_attention.py:206-344 (stases/Matterformer), the quantity the
reference's Triton backward (triton_simplicial_attention.py:332-782) computes.

Bars: fp32 operands 1e-4 (the reference's GPU parity bar,
tests/test_simplicial_attention.py:890-896 and :1000-1020); 16-bit operands
normwise relative error <= 2e-2 per gradient against float64 on the same
16-bit-rounded inputs; two runs on the same inputs bitwise identical.
"""

import numpy as np
import pytest
import torch

import matterformer_amd.hip_simplicial_attention as hsa
from matterformer_amd.hip_simplicial_attention import (
    hip_simplicial_attention_backward,
    hip_simplicial_attention_forward,
)
from matterformer_amd.simplicial_types import (
    SimplicialAttentionMask,
    SimplicialFactorizedBias,
    simplicial_attention_torch_from_projected,
)
from matterformer_amd.workloads import random_simplicial, simplicial_workload

pytestmark = pytest.mark.gpu

GRAD_NAMES = ("dq", "dk1", "dv1", "dk2", "dv2", "du", "dv_bias", "dw", "dgate")


def rel_err(got, ref):
    got = np.asarray(got, dtype=np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


def logit_std(D):
    return (4.0 / D) ** (1.0 / 6.0)


def fp64_grads(ops, qv, pkv, pv, go, bias=None):
    """float64 autograd of the torch path on the CPU: (out, [dq, dk1, dv1, dk2, dv2, du, dv, dw, dgate])."""
    leaves = [t.detach().double().cpu().requires_grad_(True) for t in ops]
    bleaves = [t.detach().double().cpu().requires_grad_(True) for t in bias] if bias is not None else []
    mask = SimplicialAttentionMask(query_valid=qv.cpu(), pair_key_valid=pkv.cpu(),
                                   pair_valid=None if pv is None else pv.cpu())
    fb = SimplicialFactorizedBias(*bleaves) if bias is not None else None
    out = simplicial_attention_torch_from_projected(*leaves, attention_mask=mask, factorized_bias=fb, chunk_size=64)
    (out * go.double().cpu()).sum().backward()
    return out.detach().numpy(), [t.grad.numpy() for t in leaves + bleaves]


def hip_grads(ops, qv, pkv, pv, go, precision, bias=None, need=True):
    kw = {}
    if bias is not None:
        kw = dict(u=bias[0], v_bias=bias[1], w=bias[2], gate=bias[3])
    out, lse, out32 = hip_simplicial_attention_forward(*ops, query_valid=qv, pair_key_valid=pkv, pair_valid=pv,
                                                       precision=precision, **kw)
    res = hip_simplicial_attention_backward(
        go, *ops, out32, lse, query_valid=qv, pair_key_valid=pkv, pair_valid=pv, precision=precision,
        need_du=need, need_dv_bias=need, need_dw=need, need_dgate=need, **kw)
    torch.cuda.synchronize()
    assert hsa.last_backward_impl == "hip"
    return out32, [r for r in res[:9]]


SHAPES = [
    # (B, H, N, D, counts, holes, pair_drop)
    (2, 4, 5, 8, [4, 2], None, 0.0),             # the reference's parity-test shape
    (1, 2, 7, 8, [5], None, 0.3),                # pair_valid (reference all-features shape)
    (3, 2, 29, 32, [29, 17, 9], [(0, 3)], 0.0),  # config-1 sized, a key hole
    (2, 2, 70, 64, [70, 41], None, 0.1),         # two column blocks + pair mask
    (2, 1, 150, 64, [150, 64], [(1, 5)], 0.0),   # three column blocks
    (2, 2, 33, 128, [33, 16], None, 0.0),        # head_dim 128 (4-wave instantiation)
    (2, 2, 24, 20, [24, 11], [(1, 5)], 0.0),     # head_dim 20, padded to 32 inside
    (3, 2, 16, 16, [16, 1, 0], None, 0.0),       # one-atom and empty molecules
]


def _case(shape, seed, dtype, device):
    B, H, N, D, counts, holes, drop = shape
    case = random_simplicial(B, H, N, D, seed=seed, counts=counts, holes=holes, pair_drop=drop, std=logit_std(D))
    q, k1, v1, k2, v2, qv, pkv, pv = case
    gen = torch.Generator().manual_seed(seed + 1)
    go = torch.randn(B, H, N, D, generator=gen)
    ops_cpu = [t.to(dtype) for t in (q, k1, v1, k2, v2)]
    ops = [t.to(device) for t in ops_cpu]
    return ops_cpu, ops, qv, pkv, pv, go.to(dtype)


@pytest.mark.parametrize("with_bias", [False, True], ids=["nobias", "bias"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"B{s[0]}H{s[1]}N{s[2]}D{s[3]}")
def test_fp32_gradients_match_fp64(cuda, shape, with_bias):
    B, H, N, D = shape[:4]
    ops_cpu, ops, qv, pkv, pv, go = _case(shape, seed=N * 7 + D, dtype=torch.float32, device=cuda)
    bias = None
    if with_bias:
        gen = torch.Generator().manual_seed(N + 3)
        bias = [torch.randn(B, H, N, N, generator=gen) * 0.5 for _ in range(3)] + [torch.randn(B, H, N, generator=gen)]
    out32, got = hip_grads(ops, qv.to(cuda), pkv.to(cuda), None if pv is None else pv.to(cuda), go.to(cuda),
                           "ieee_fp32", bias=None if bias is None else [t.to(cuda) for t in bias])
    _, ref = fp64_grads(ops_cpu, qv, pkv, pv, go, bias=bias)
    names = GRAD_NAMES if with_bias else GRAD_NAMES[:5]
    for name, g, r in zip(names, got, ref):
        np.testing.assert_allclose(g.cpu().numpy(), r, rtol=1e-4, atol=1e-4, err_msg=name)
    if not with_bias:
        assert all(x is None for x in got[5:])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("shape", SHAPES[2:6], ids=lambda s: f"B{s[0]}H{s[1]}N{s[2]}D{s[3]}")
def test_16bit_gradients_match_fp64(cuda, shape, dtype):
    B, H, N, D = shape[:4]
    ops_cpu, ops, qv, pkv, pv, go = _case(shape, seed=N * 11 + D, dtype=dtype, device=cuda)
    gen = torch.Generator().manual_seed(N + 5)
    bias = [(torch.randn(B, H, N, N, generator=gen) * 0.5).to(dtype) for _ in range(3)] + \
           [torch.randn(B, H, N, generator=gen).to(dtype)]
    out32, got = hip_grads(ops, qv.to(cuda), pkv.to(cuda), None if pv is None else pv.to(cuda), go.to(cuda),
                           "bf16_tc", bias=[t.to(cuda) for t in bias])
    _, ref = fp64_grads(ops_cpu, qv, pkv, pv, go, bias=bias)
    for name, g, r in zip(GRAD_NAMES, got, ref):
        assert g.dtype == dtype, name
        assert rel_err(g.float().cpu().numpy(), r) <= 2e-2, name


def test_bf16_gradients_with_cancelling_value_products(cuda):
    """bf16 operands whose values are nearly constant (v = 1 + 0.03 z) under a logit spread of std 2: the value
    product dP_ijk = go_i . (v1_j (.) v2_k) then differs from delta_i = go_i . out_i by a few percent of itself,
    so dS = P (dP - delta) cancels about 5 bits.  Rounding the dP operand go (.) v once to bf16 gives 6-16 %
    gradient errors here (float64 simulation of that rounding); the kernel carries it as bf16 hi + lo.
    Bar: 2e-2 per gradient against float64 autograd on the same bf16 inputs."""
    B, H, N, D = 2, 2, 29, 64
    counts = [29, 20]
    case = random_simplicial(B, H, N, D, seed=91, counts=counts, std=logit_std(D))
    q, k1, v1, k2, v2, qv, pkv, pv = case
    gen = torch.Generator().manual_seed(92)
    v1 = 1.0 + 0.03 * torch.randn(B, H, N, D, generator=gen)
    v2 = 1.0 + 0.03 * torch.randn(B, H, N, D, generator=gen)
    go = torch.randn(B, H, N, D, generator=gen).to(torch.bfloat16)
    ops_cpu = [t.to(torch.bfloat16) for t in (q, k1, v1, k2, v2)]
    _, got = hip_grads([t.to(cuda) for t in ops_cpu], qv.to(cuda), pkv.to(cuda), None, go.to(cuda), "bf16_tc")
    _, ref = fp64_grads(ops_cpu, qv, pkv, None, go)
    errs = {name: rel_err(g.float().cpu().numpy(), r) for name, g, r in zip(GRAD_NAMES, got[:5], ref)}
    print("cancelling value products, bf16 gradient errors:", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    for name, e in errs.items():
        assert e <= 2e-2, (name, e)


def test_qm9_config_gradients_whole_batch(cuda):
    """Config 1 (fp32, 128 molecules): every gradient against float64 autograd at 1e-4."""
    w = simplicial_workload("qm9")
    B, H, N, D = w.shape
    gen = torch.Generator().manual_seed(55)
    go = torch.randn(B, H, N, D, generator=gen)
    ops_cpu = [w.q, w.k1, w.v1, w.k2, w.v2]
    out32, got = hip_grads([t.to(cuda) for t in ops_cpu], w.query_valid.to(cuda), w.pair_key_valid.to(cuda), None,
                           go.to(cuda), "ieee_fp32")
    _, ref = fp64_grads(ops_cpu, w.query_valid, w.pair_key_valid, None, go)
    for name, g, r in zip(GRAD_NAMES, got[:5], ref):
        np.testing.assert_allclose(g.cpu().numpy(), r, rtol=1e-4, atol=1e-4, err_msg=name)


@pytest.mark.parametrize("with_bias", [False, True], ids=["nobias", "bias"])
def test_geom_config_gradients_every_molecule(cuda, with_bias):
    """Config 2 (bf16, 64 molecules of 10-72 atoms padded to 181), without a bias (the pair-formulation kernel)
    and with a factorized bias (the ownership kernel): the batched HIP gradients of each molecule against
    float64 autograd over that molecule's atoms, 2e-2 per gradient."""
    w = simplicial_workload("geom")
    B, H, N, D = w.shape
    gen = torch.Generator().manual_seed(56)
    go = torch.randn(B, H, N, D, generator=gen).to(torch.bfloat16)
    bias = [(torch.randn(B, H, N, N, generator=gen) * 0.5).to(torch.bfloat16) for _ in range(3)] + \
           [torch.randn(B, H, N, generator=gen).to(torch.bfloat16)]
    if not with_bias:
        bias = None
    ops_cpu = [t.to(torch.bfloat16) for t in (w.q, w.k1, w.v1, w.k2, w.v2)]
    _, got = hip_grads([t.to(cuda) for t in ops_cpu], w.query_valid.to(cuda), w.pair_key_valid.to(cuda), None,
                       go.to(cuda), "bf16_tc", bias=None if bias is None else [t.to(cuda) for t in bias])
    got = [g.float().cpu() for g in got if g is not None]
    worst = {}
    for b in range(B):
        n = int(w.counts[b])
        ones = torch.ones(1, n, dtype=torch.bool)
        sl = [t[b:b + 1, :, :n] for t in ops_cpu]
        bsl = None if bias is None else [t[b:b + 1, :, :n, :n] for t in bias[:3]] + [bias[3][b:b + 1, :, :n]]
        _, ref = fp64_grads(sl, ones, ones, None, go[b:b + 1, :, :n], bias=bsl)
        for idx, (name, r) in enumerate(zip(GRAD_NAMES, ref)):
            g = got[idx][b:b + 1, :, :n]
            if name in ("du", "dv_bias", "dw"):
                g = g[..., :n]
            e = rel_err(g.numpy(), r)
            worst[name] = max(worst.get(name, 0.0), e)
            assert e <= 2e-2, (b, name, e)
        # gradients of padded rows stay zero
        assert torch.count_nonzero(got[0][b, :, n:]) == 0 and torch.count_nonzero(got[1][b, :, n:]) == 0
    print("worst per-molecule relative error:", {k: f"{v:.2e}" for k, v in worst.items()}, flush=True)


@pytest.mark.parametrize("with_bias", [False, True], ids=["nobias", "bias"])
def test_backward_is_bitwise_deterministic(cuda, with_bias):
    """Two backward calls on the same inputs (config-2 sized, with and without a bias) give identical bits."""
    w = simplicial_workload("geom", batch=16)
    B, H, N, D = w.shape
    gen = torch.Generator().manual_seed(57)
    go = torch.randn(B, H, N, D, generator=gen).to(torch.bfloat16).to(cuda)
    bias = [(torch.randn(B, H, N, N, generator=gen) * 0.5).to(torch.bfloat16).to(cuda) for _ in range(3)] + \
           [torch.randn(B, H, N, generator=gen).to(torch.bfloat16).to(cuda)]
    if not with_bias:
        bias = None
    ops = [t.to(torch.bfloat16).to(cuda) for t in (w.q, w.k1, w.v1, w.k2, w.v2)]
    qv, pkv = w.query_valid.to(cuda), w.pair_key_valid.to(cuda)
    _, first = hip_grads(ops, qv, pkv, None, go, "bf16_tc", bias=bias)
    _, second = hip_grads(ops, qv, pkv, None, go, "bf16_tc", bias=bias)
    for name, a, b in zip(GRAD_NAMES, first, second):
        assert (a is None) == (b is None), name
        assert a is None or torch.equal(a, b), name


def test_only_requested_bias_gradients_are_returned(cuda):
    shape = (2, 2, 12, 16, [12, 7], None, 0.0)
    B, H, N, D = shape[:4]
    ops_cpu, ops, qv, pkv, pv, go = _case(shape, seed=3, dtype=torch.float32, device=cuda)
    bias = [torch.randn(B, H, N, N, device=cuda) for _ in range(3)] + [torch.randn(B, H, N, device=cuda)]
    out, lse, out32 = hip_simplicial_attention_forward(*ops, query_valid=qv.to(cuda), pair_key_valid=pkv.to(cuda),
                                                       pair_valid=None, precision="ieee_fp32", u=bias[0],
                                                       v_bias=bias[1], w=bias[2], gate=bias[3])
    res = hip_simplicial_attention_backward(
        go.to(cuda), *ops, out32, lse, query_valid=qv.to(cuda), pair_key_valid=pkv.to(cuda), pair_valid=None,
        u=bias[0], v_bias=bias[1], w=bias[2], gate=bias[3], precision="ieee_fp32",
        need_du=False, need_dv_bias=True, need_dw=False, need_dgate=True)
    assert hsa.last_backward_impl == "hip"
    assert res[5] is None and res[7] is None and res[6] is not None and res[8] is not None


def test_low_rank_terms_run_on_the_kernel(cuda):
    """Angle / message gradients come from mf_simplicial_bwd, not from a torch recompute."""
    B, H, N, D = 1, 2, 6, 8
    q, k1, v1, k2, v2 = (torch.randn(B, H, N, D, device=cuda) for _ in range(5))
    ones = torch.ones(B, N, dtype=torch.bool, device=cuda)
    al, ar = (torch.randn(B, H, N, N, 3, device=cuda) for _ in range(2))
    ag = torch.randn(B, H, N, device=cuda)
    out, lse, out32 = hip_simplicial_attention_forward(q, k1, v1, k2, v2, query_valid=ones, pair_key_valid=ones,
                                                       pair_valid=None, angle_left=al, angle_right=ar, angle_gate=ag,
                                                       precision="ieee_fp32")
    res = hip_simplicial_attention_backward(torch.randn_like(q), q, k1, v1, k2, v2, out32, lse, query_valid=ones,
                                            pair_key_valid=ones, pair_valid=None, angle_left=al, angle_right=ar,
                                            angle_gate=ag, precision="ieee_fp32")
    assert hsa.last_backward_impl == "hip"
    assert res[9] is not None and res[11] is not None


def _abi_bwd(ops, go, out32, lse, qv, pkv, grads_dtype, bias=None):
    """mf_simplicial_bwd through the C ABI; gradient buffers filled with NaN (bf16) or zeros (fp32, the
    caller's fill that the fp32 contract asks for); with a bf16 factorized bias also du, dv_bias, dw, dgate
    (the same dtype and fill)."""
    from matterformer_amd import _native

    B, H, N, D = ops[0].shape
    dev = ops[0].device
    lib = _native.lib()
    nbytes = int(lib.mf_simplicial_bwd_workspace_size(B, H, N, D, 0))
    ws = torch.empty(max(nbytes, 16), device=dev, dtype=torch.uint8)
    if grads_dtype == torch.bfloat16:
        grads = [torch.full((B, H, N, D), float("nan"), device=dev, dtype=torch.bfloat16) for _ in range(5)]
    else:
        grads = [torch.zeros(B, H, N, D, device=dev) for _ in range(5)]
    qb, pb = qv.to(torch.bool).contiguous(), pkv.to(torch.bool).contiguous()
    extra = {}
    if bias is not None:
        if grads_dtype == torch.bfloat16:
            bgrads = [torch.full(s, float("nan"), device=dev, dtype=torch.bfloat16)
                      for s in ((B, H, N, N),) * 3 + ((B, H, N),)]
        else:
            bgrads = [torch.zeros(B, H, N, N, device=dev) for _ in range(3)] + [torch.zeros(B, H, N, device=dev)]
        extra = dict(bias_u=bias[0].data_ptr(), bias_v=bias[1].data_ptr(), bias_w=bias[2].data_ptr(),
                     bias_gate=bias[3].data_ptr(), bias_dtype=_native.dtype_code(bias[0].dtype),
                     du=bgrads[0].data_ptr(), dv_bias=bgrads[1].data_ptr(), dw=bgrads[2].data_ptr(),
                     dgate=bgrads[3].data_ptr())
        grads = grads + bgrads
    args = _native.MfSimplicialBwdArgs(
        q=ops[0].data_ptr(), k1=ops[1].data_ptr(), v1=ops[2].data_ptr(), k2=ops[3].data_ptr(), v2=ops[4].data_ptr(),
        grad_out=go.data_ptr(), out=out32.data_ptr(), lse=lse.float().contiguous().data_ptr(),
        query_valid=qb.data_ptr(), pair_key_valid=pb.data_ptr(), pair_valid=None,
        grad_dtype=_native.dtype_code(torch.bfloat16), dq=grads[0].data_ptr(), dk1=grads[1].data_ptr(),
        dv1=grads[2].data_ptr(), dk2=grads[3].data_ptr(), dv2=grads[4].data_ptr(), batch=B, heads=H, tokens=N,
        head_dim=D, dtype=_native.dtype_code(torch.bfloat16), grads_dtype=_native.dtype_code(grads_dtype),
        workspace=ws.data_ptr(), workspace_bytes=nbytes, **extra)
    with torch.cuda.device(dev):
        _native.check(lib.mf_simplicial_bwd(args, _native.current_stream(dev)), "mf_simplicial_bwd")
    torch.cuda.synchronize()
    return grads


@pytest.mark.parametrize("with_bias", [False, True], ids=["nobias", "bias"])
@pytest.mark.parametrize("counts", [[70, 41, 0, 12], [150, 64, 1, 33]], ids=["pair_only", "with_ownership"])
def test_bf16_gradients_written_in_full(cuda, counts, with_bias):
    """grads_dtype bf16: every element of the gradients (the bias gradients too) is written (buffers start as
    NaN; padded rows and entries, and a molecule without valid queries, come back 0), and the values are the
    fp32-gradient call's rounded to bf16 (both paths form the same fp32 sums).  The second case has a 150-atom
    molecule (ownership kernel) beside pair-kernel molecules, one of them split in two halves; the 70-atom
    molecule runs its query tiles in two passes when there is a bias."""
    B, H, N, D = len(counts), 2, max(counts) + 3, 64
    case = random_simplicial(B, H, N, D, seed=71, counts=counts, std=logit_std(D))
    q, k1, v1, k2, v2, qv, pkv, pv = case
    qv = qv.clone()
    qv[2] = False  # molecule 2: keys but no valid query
    gen = torch.Generator().manual_seed(72)
    go = torch.randn(B, H, N, D, generator=gen).to(torch.bfloat16).to(cuda)
    ops = [t.to(torch.bfloat16).to(cuda).contiguous() for t in (q, k1, v1, k2, v2)]
    qv, pkv = qv.to(cuda), pkv.to(cuda)
    bias, kw = None, {}
    if with_bias:
        bias = [(torch.randn(B, H, N, N, generator=gen) * 0.5).to(torch.bfloat16).to(cuda) for _ in range(3)] + \
               [torch.randn(B, H, N, generator=gen).to(torch.bfloat16).to(cuda)]
        kw = dict(u=bias[0], v_bias=bias[1], w=bias[2], gate=bias[3])
    out, lse, out32 = hip_simplicial_attention_forward(*ops, query_valid=qv, pair_key_valid=pkv, pair_valid=None,
                                                       precision="bf16_tc", **kw)
    g16 = _abi_bwd(ops, go, out32, lse, qv, pkv, torch.bfloat16, bias=bias)
    g32 = _abi_bwd(ops, go, out32, lse, qv, pkv, torch.float32, bias=bias)
    for name, a, r in zip(GRAD_NAMES, g16, g32):
        assert not torch.isnan(a).any(), name
        assert torch.equal(a, r.to(torch.bfloat16)), name
    # padded rows, and every row of molecule 2, are zero
    qvc, pkvc = qv.cpu(), pkv.cpu()
    for b in range(B):
        rows_q = ~qvc[b] if b != 2 else torch.ones(N, dtype=torch.bool)
        rows_k = ~pkvc[b] if b != 2 else torch.ones(N, dtype=torch.bool)
        assert not g16[0][b][:, rows_q.to(cuda)].any()
        for g in g16[1:5]:
            assert not g[b][:, rows_k.to(cuda)].any()
        if with_bias:  # du, dv_bias at padded (query, key), dw at padded (key, key), dgate at padded queries
            rq, rk = rows_q.to(cuda), rows_k.to(cuda)
            for g in g16[5:7]:
                assert not g[b][:, rq, :].any() and not g[b][:, :, rk].any()
            assert not g16[7][b][:, rk, :].any() and not g16[7][b][:, :, rk].any()
            assert not g16[8][b][:, rq].any()


def test_pair_path_bias_gradients_with_masking_scale_terms(cuda):
    """bf16 operands, pair formulation with a factorized bias whose w carries -30000 on a fifth of the pairs
    (positive gates: those pairs' P underflows to 0, as under an additive mask) beside ordinary terms; one
    molecule of 70 atoms (split in two halves, query tiles in two passes) and one of 41.  Every gradient
    against float64 autograd on the same rounded inputs, 2e-2."""
    B, H, N, D = 2, 2, 70, 64
    case = random_simplicial(B, H, N, D, seed=81, counts=[70, 41], std=logit_std(D))
    q, k1, v1, k2, v2, qv, pkv, pv = case
    gen = torch.Generator().manual_seed(82)
    go = torch.randn(B, H, N, D, generator=gen).to(torch.bfloat16)
    u, v, w = (torch.randn(B, H, N, N, generator=gen) * 0.5 for _ in range(3))
    w[torch.rand(B, H, N, N, generator=gen) < 0.2] = -30000.0
    gate = torch.rand(B, H, N, generator=gen) + 0.5
    bias = [t.to(torch.bfloat16) for t in (u, v, w, gate)]
    ops_cpu = [t.to(torch.bfloat16) for t in (q, k1, v1, k2, v2)]
    _, got = hip_grads([t.to(cuda) for t in ops_cpu], qv.to(cuda), pkv.to(cuda), None, go.to(cuda), "bf16_tc",
                       bias=[t.to(cuda) for t in bias])
    _, ref = fp64_grads(ops_cpu, qv, pkv, None, go, bias=bias)
    errs = {}
    for name, g, r in zip(GRAD_NAMES, got, ref):
        errs[name] = rel_err(g.float().cpu().numpy(), r)
    print("relative errors:", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    for name, e in errs.items():
        assert e <= 2e-2, (name, e)
