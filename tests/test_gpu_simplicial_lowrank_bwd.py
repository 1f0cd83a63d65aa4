"""GPU parity of the low-rank angle and message gradients of mf_simplicial_bwd against float64 autograd.

The terms are the reference's SimplicialLowRankAngleResidual (S += gate_i R^-1/2 sum_r L_ijr R_ikr) and
SimplicialLowRankMessageResidual (out_i += sum_r c_ir basis_r, c_ir = R^-1/2 sum_jk P_ijk L_ijr R_ikr),
simplicial_attention.py:50-104,330-337; their gradients are those of triton_simplicial_attention.py:488-515,
575-782 (dangle_left / right / gate, dmessage_left / right / basis), which the reference accumulates with
atomics and this kernel by ownership.  The checker is autograd of the product's torch path in float64 on the
CPU (the path is bit-identical to the reference's torch path on every committed fixture, including the
bias + angle + message one).

Bars: fp32 operands 1e-4 (rtol and atol, the reference's GPU parity bar); 16-bit operands 2e-2 normwise per
gradient against float64 on the same 16-bit-rounded inputs; two runs bitwise identical.
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
    SimplicialLowRankAngleResidual,
    SimplicialLowRankMessageResidual,
    simplicial_attention_torch_from_projected,
)
from matterformer_amd.workloads import random_simplicial, simplicial_workload

pytestmark = pytest.mark.gpu

NAMES = ("dq", "dk1", "dv1", "dk2", "dv2", "du", "dv_bias", "dw", "dgate",
         "dangle_left", "dangle_right", "dangle_gate", "dmessage_left", "dmessage_right", "dmessage_basis")


def rel_err(got, ref):
    got = np.asarray(got, dtype=np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


def logit_std(D):
    return (4.0 / D) ** (1.0 / 6.0)


def make_terms(B, H, N, D, seed, *, bias, ra, rm):
    gen = torch.Generator().manual_seed(seed)
    t = {}
    if bias:
        t["bias"] = [torch.randn(B, H, N, N, generator=gen) * 0.5 for _ in range(3)] + \
                    [torch.randn(B, H, N, generator=gen)]
    if ra:
        t["angle"] = [torch.randn(B, H, N, N, ra, generator=gen) * 0.7 for _ in range(2)] + \
                     [torch.randn(B, H, N, generator=gen)]
    if rm:
        t["message"] = [torch.randn(B, H, N, N, rm, generator=gen) for _ in range(2)] + \
                       [torch.randn(H, rm, D, generator=gen) * D ** -0.5]
    return t


def fp64_grads(ops, qv, pkv, pv, go, terms, batch=None):
    """float64 autograd of the torch path on the CPU; gradients in NAMES order (None where absent)."""
    sl = (lambda x: x) if batch is None else batch
    leaves = [sl(t).detach().double().cpu().requires_grad_(True) for t in ops]
    groups = {k: [t.detach().double().cpu().requires_grad_(True) for t in v] for k, v in terms.items()}
    mask = SimplicialAttentionMask(query_valid=qv.cpu(), pair_key_valid=pkv.cpu(),
                                   pair_valid=None if pv is None else pv.cpu())
    fb = SimplicialFactorizedBias(*groups["bias"]) if "bias" in groups else None
    ar = SimplicialLowRankAngleResidual(*groups["angle"]) if "angle" in groups else None
    mr = SimplicialLowRankMessageResidual(*groups["message"][:2]) if "message" in groups else None
    out = simplicial_attention_torch_from_projected(
        *leaves, attention_mask=mask, factorized_bias=fb, angle_residual=ar, message_residual=mr,
        message_basis=groups["message"][2] if "message" in groups else None, chunk_size=64)
    (out * go.double().cpu()).sum().backward()
    res = [t.grad.numpy() for t in leaves]
    for key in ("bias", "angle", "message"):
        n = 4 if key == "bias" else 3
        res += [t.grad.numpy() for t in groups[key]] if key in groups else [None] * n
    return res


def hip_grads(ops, qv, pkv, pv, go, precision, terms):
    kw = {}
    if "bias" in terms:
        kw.update(zip(("u", "v_bias", "w", "gate"), terms["bias"]))
    if "angle" in terms:
        kw.update(zip(("angle_left", "angle_right", "angle_gate"), terms["angle"]))
    if "message" in terms:
        kw.update(zip(("message_left", "message_right", "message_basis"), terms["message"]))
    out, lse, out32 = hip_simplicial_attention_forward(*ops, query_valid=qv, pair_key_valid=pkv, pair_valid=pv,
                                                       precision=precision, **kw)
    res = hip_simplicial_attention_backward(go, *ops, out32, lse, query_valid=qv, pair_key_valid=pkv, pair_valid=pv,
                                            precision=precision, **kw)
    torch.cuda.synchronize()
    assert hsa.last_backward_impl == "hip"
    return list(res)


def _to(terms, device, dtype=None):
    return {k: [t.to(device) if dtype is None else t.to(device, dtype) for t in v] for k, v in terms.items()}


CASES = [
    # (B, H, N, D, counts, holes, pair_drop, bias, Ra, Rm)
    (3, 2, 29, 32, [29, 17, 9], [(0, 3)], 0.0, False, 5, 0),     # config-1 sized, angle only, rank 5
    (3, 2, 29, 32, [29, 17, 9], None, 0.0, True, 0, 16),         # message only, rank 16, with the bias
    (2, 2, 29, 32, [29, 20], None, 0.2, True, 16, 5),            # both terms, pair_valid
    (2, 2, 70, 64, [70, 41], None, 0.0, False, 33, 64),          # two column blocks, ranks 33 and 64
    (2, 1, 40, 128, [40, 13], [(1, 2)], 0.0, True, 8, 12),       # head_dim 128
    (3, 2, 16, 20, [16, 1, 0], None, 0.0, False, 3, 7),          # head_dim 20, one-atom and empty molecules
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"N{c[2]}D{c[3]}Ra{c[8]}Rm{c[9]}{'b' if c[7] else ''}")
def test_fp32_low_rank_gradients_match_fp64(cuda, case):
    B, H, N, D, counts, holes, drop, bias, ra, rm = case
    q, k1, v1, k2, v2, qv, pkv, pv = random_simplicial(B, H, N, D, seed=N * 3 + ra + rm, counts=counts,
                                                       holes=holes, pair_drop=drop, std=logit_std(D))
    gen = torch.Generator().manual_seed(N + ra * 7 + rm)
    go = torch.randn(B, H, N, D, generator=gen)
    terms = make_terms(B, H, N, D, seed=ra * 31 + rm, bias=bias, ra=ra, rm=rm)
    ops = [q, k1, v1, k2, v2]
    got = hip_grads([t.to(cuda) for t in ops], qv.to(cuda), pkv.to(cuda), None if pv is None else pv.to(cuda),
                    go.to(cuda), "ieee_fp32", _to(terms, cuda))
    ref = fp64_grads(ops, qv, pkv, pv, go, terms)
    for name, g, r in zip(NAMES, got, ref):
        if r is None:
            assert g is None, name
            continue
        np.testing.assert_allclose(g.cpu().numpy(), r, rtol=1e-4, atol=1e-4, err_msg=name)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("ra,rm", [(16, 16), (33, 5)])
def test_16bit_low_rank_gradients_match_fp64(cuda, dtype, ra, rm):
    B, H, N, D = 2, 2, 70, 64
    q, k1, v1, k2, v2, qv, pkv, pv = random_simplicial(B, H, N, D, seed=ra + rm, counts=[70, 41], std=logit_std(D))
    gen = torch.Generator().manual_seed(ra * rm)
    go = torch.randn(B, H, N, D, generator=gen).to(dtype)
    terms = make_terms(B, H, N, D, seed=ra + 2 * rm, bias=True, ra=ra, rm=rm)
    terms["bias"] = [t.to(dtype) for t in terms["bias"]]
    ops = [t.to(dtype) for t in (q, k1, v1, k2, v2)]
    got = hip_grads([t.to(cuda) for t in ops], qv.to(cuda), pkv.to(cuda), None, go.to(cuda), "bf16_tc",
                    _to(terms, cuda))
    ref = fp64_grads(ops, qv, pkv, None, go, terms)
    errs = {n: rel_err(g.float().cpu().numpy(), r) for n, g, r in zip(NAMES, got, ref) if r is not None}
    print(f"{dtype} ranks {ra}/{rm}:", {k: f"{v:.1e}" for k, v in errs.items()}, flush=True)
    for name, e in errs.items():
        assert e <= 2e-2, (name, e)


def test_qm9_config_low_rank_gradients_whole_batch(cuda):
    """Config 1 (fp32, 128 molecules, N = 29, D = 32) with an angle term of rank 5 and a message term of
    rank 33: every gradient against float64 autograd at 1e-4."""
    w = simplicial_workload("qm9")
    B, H, N, D = w.shape
    gen = torch.Generator().manual_seed(58)
    go = torch.randn(B, H, N, D, generator=gen)
    terms = make_terms(B, H, N, D, seed=59, bias=False, ra=5, rm=33)
    ops = [w.q, w.k1, w.v1, w.k2, w.v2]
    got = hip_grads([t.to(cuda) for t in ops], w.query_valid.to(cuda), w.pair_key_valid.to(cuda), None, go.to(cuda),
                    "ieee_fp32", _to(terms, cuda))
    ref = fp64_grads(ops, w.query_valid, w.pair_key_valid, None, go, terms)
    for name, g, r in zip(NAMES, got, ref):
        if r is not None:
            np.testing.assert_allclose(g.cpu().numpy(), r, rtol=1e-4, atol=1e-4, err_msg=name)


def test_geom_config_low_rank_gradients_every_molecule(cuda):
    """Config 2 (bf16, 64 molecules up to 181 atoms, D = 64) with the factorized bias, an angle term of rank 16
    and a message term of rank 16: each molecule's gradients against float64 autograd over its atoms, 2e-2
    per gradient (dmessage_basis, a sum over the whole batch, against the sum of the molecules' references)."""
    w = simplicial_workload("geom")
    B, H, N, D = w.shape
    gen = torch.Generator().manual_seed(60)
    go = torch.randn(B, H, N, D, generator=gen).to(torch.bfloat16)
    terms = make_terms(B, H, N, D, seed=61, bias=True, ra=16, rm=16)
    terms["bias"] = [t.to(torch.bfloat16) for t in terms["bias"]]
    ops = [t.to(torch.bfloat16) for t in (w.q, w.k1, w.v1, w.k2, w.v2)]
    got = hip_grads([t.to(cuda) for t in ops], w.query_valid.to(cuda), w.pair_key_valid.to(cuda), None, go.to(cuda),
                    "bf16_tc", _to(terms, cuda))
    got = [g.float().cpu() for g in got]
    worst = {}
    basis_ref = np.zeros(got[14].shape)
    for b in range(B):
        n = int(w.counts[b])
        ones = torch.ones(1, n, dtype=torch.bool)
        sl = [t[b:b + 1, :, :n] for t in ops]
        tb = {"bias": [t[b:b + 1, :, :n, :n] for t in terms["bias"][:3]] + [terms["bias"][3][b:b + 1, :, :n]],
              "angle": [t[b:b + 1, :, :n, :n] for t in terms["angle"][:2]] + [terms["angle"][2][b:b + 1, :, :n]],
              "message": [t[b:b + 1, :, :n, :n] for t in terms["message"][:2]] + [terms["message"][2]]}
        ref = fp64_grads(sl, ones, ones, None, go[b:b + 1, :, :n], tb)
        basis_ref += ref[14]
        for idx, (name, r) in enumerate(zip(NAMES[:14], ref[:14])):
            g = got[idx][b:b + 1, :, :n]
            if name in ("du", "dv_bias", "dw", "dangle_left", "dangle_right", "dmessage_left", "dmessage_right"):
                g = g[:, :, :, :n]
            e = rel_err(g.numpy(), r)
            worst[name] = max(worst.get(name, 0.0), e)
            assert e <= 2e-2, (b, name, e)
    e = rel_err(got[14].numpy(), basis_ref)
    worst["dmessage_basis"] = e
    print("worst per-molecule relative error:", {k: f"{v:.2e}" for k, v in worst.items()}, flush=True)
    assert e <= 2e-2


def test_low_rank_backward_is_bitwise_deterministic(cuda):
    B, H, N, D = 4, 2, 61, 64
    q, k1, v1, k2, v2, qv, pkv, pv = random_simplicial(B, H, N, D, seed=7, counts=[61, 40, 33, 12], std=logit_std(D))
    terms = _to(make_terms(B, H, N, D, seed=8, bias=True, ra=16, rm=12), cuda)
    go = torch.randn(B, H, N, D, generator=torch.Generator().manual_seed(9)).to(cuda)
    ops = [t.to(cuda) for t in (q, k1, v1, k2, v2)]
    first = hip_grads(ops, qv.to(cuda), pkv.to(cuda), None, go, "ieee_fp32", terms)
    second = hip_grads(ops, qv.to(cuda), pkv.to(cuda), None, go, "ieee_fp32", terms)
    for name, a, b in zip(NAMES, first, second):
        assert torch.equal(a, b), name
