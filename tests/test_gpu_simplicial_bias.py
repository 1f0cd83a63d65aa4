"""GPU parity of the fused optional terms of mf_simplicial_fwd: factorized bias, low-rank angle, low-rank message.

Reference semantics: triton_simplicial_attention.py:244-279,305-326 and
simplicial_attention.py:18-104,330-337 (stases/Matterformer).  The checker is
the float64 brute force of oracle/simplicial.py, itself pinned to the
reference's bias + angle + message fixture (tests/test_oracle_simplicial.py).

Tolerances as for the plain forward: fp32 operands with ieee_fp32 precision
1e-4 (the reference's own parity bar, tests/test_simplicial_attention.py:1017),
16-bit operands normwise relative error <= 2e-2 against float64 on the same
16-bit-rounded inputs, and additionally every valid query row within 3e-2 of
its own norm, so a few wrong rows cannot hide in the normwise figure (the
worst row measured over every case here is 2.1e-2, bf16 with the low-rank
message term at N = 130; fp16 cases stay below 3e-3).
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from matterformer_amd.hip_simplicial_attention import hip_simplicial_attention_forward
from matterformer_amd.simplicial_attention import SimplicialAttention
from matterformer_amd.simplicial_types import (
    SimplicialAttentionMask,
    SimplicialFactorizedBias,
    SimplicialLowRankAngleResidual,
    SimplicialLowRankMessageResidual,
    simplicial_attention_torch_from_projected,
)
from matterformer_amd.workloads import random_simplicial, simplicial_workload
from oracle.simplicial import brute_force_fp64

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def rel_err(got, ref):
    got = np.asarray(got, dtype=np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


def row_errors(got, ref, qv):
    """Per valid (b, h, i) row: |got - ref| / max(|ref|, 1e-3 * typical row norm)."""
    got = np.asarray(got, dtype=np.float64)
    rows = qv.numpy().astype(bool)[:, None, :].repeat(got.shape[1], 1)  # [B, H, N]
    diff = np.linalg.norm(got - ref, axis=-1)[rows]
    norm = np.linalg.norm(ref, axis=-1)[rows]
    floor = 1e-3 * max(float(np.median(norm)), 1e-30)
    return diff / np.maximum(norm, floor)


def make_terms(B, H, N, D, seed, *, bias=True, angle_rank=0, message_rank=0, scale=0.5):
    gen = torch.Generator().manual_seed(seed)
    terms = {}
    if bias:
        terms["bias"] = [torch.randn(B, H, N, N, generator=gen) * scale for _ in range(3)] + \
                        [torch.randn(B, H, N, generator=gen)]
    if angle_rank:
        terms["angle"] = [torch.randn(B, H, N, N, angle_rank, generator=gen) * scale for _ in range(2)] + \
                         [torch.randn(B, H, N, generator=gen)]
    if message_rank:
        terms["message"] = [torch.randn(B, H, N, N, message_rank, generator=gen) for _ in range(2)] + \
                           [torch.randn(H, message_rank, D, generator=gen) * D ** -0.5]
    return terms


def run(case, terms, device, dtype, precision, bias_dtype=None):
    q, k1, v1, k2, v2, qv, pkv, pv = case
    ops = [t.to(dtype).to(device) for t in (q, k1, v1, k2, v2)]
    kw = {}
    if "bias" in terms:
        bdt = bias_dtype or dtype
        u, v, w, gate = (t.to(bdt).to(device) for t in terms["bias"])
        kw.update(u=u, v_bias=v, w=w, gate=gate)
    if "angle" in terms:
        left, right, gate = (t.to(device) for t in terms["angle"])
        kw.update(angle_left=left, angle_right=right, angle_gate=gate)
    if "message" in terms:
        left, right, basis = (t.to(device) for t in terms["message"])
        kw.update(message_left=left, message_right=right, message_basis=basis)
    out, lse, out32 = hip_simplicial_attention_forward(
        *ops, query_valid=qv.to(device), pair_key_valid=pkv.to(device),
        pair_valid=None if pv is None else pv.to(device), precision=precision, **kw)
    torch.cuda.synchronize()
    return out, lse, out32


def oracle(case, terms, dtype, bias_dtype=None):
    q, k1, v1, k2, v2, qv, pkv, pv = case
    ops = [t.to(dtype).double().numpy() for t in (q, k1, v1, k2, v2)]
    kw = {}
    if "bias" in terms:
        bdt = bias_dtype or dtype
        kw["bias"] = tuple(t.to(bdt).double().numpy() for t in terms["bias"])
    if "angle" in terms:
        kw["angle"] = tuple(t.double().numpy() for t in terms["angle"])
    if "message" in terms:
        kw["message"] = tuple(t.double().numpy() for t in terms["message"])
    return brute_force_fp64(*ops, qv.numpy(), pkv.numpy(), None if pv is None else pv.numpy(), **kw)


def logit_std(D):
    return (4.0 / D) ** (1.0 / 6.0)


# every valid query row within this fraction of its own norm (16-bit operands)
ROW_BAR = 3e-2


def test_reference_golden_bias_angle_message(cuda):
    z = np.load(GOLDEN / "simplicial_fp32_bias_angle_message.npz")
    t = {k: torch.from_numpy(z[k]).to(cuda) for k in z.files if z[k].ndim > 0}
    out, lse, out32 = hip_simplicial_attention_forward(
        t["q"], t["k1"], t["v1"], t["k2"], t["v2"], query_valid=t["query_valid"],
        pair_key_valid=t["pair_key_valid"], pair_valid=t["pair_valid"],
        u=t["u"], v_bias=t["v_bias"], w=t["w"], gate=t["gate"],
        angle_left=t["angle_left"], angle_right=t["angle_right"], angle_gate=t["angle_gate"],
        message_left=t["message_left"], message_right=t["message_right"], message_basis=t["message_basis"],
        precision="ieee_fp32")
    torch.cuda.synchronize()
    np.testing.assert_allclose(out32.cpu().numpy(), z["out"], rtol=1e-4, atol=1e-4)


SHAPES = [
    # (B, H, N, D, counts, holes, pair_drop)
    (1, 2, 7, 8, [5], None, 0.2),
    (3, 2, 29, 32, [29, 17, 9], [(0, 3)], 0.0),
    (2, 2, 70, 64, [70, 41], None, 0.1),      # more than 64 keys in one block
    (2, 1, 81, 64, [81, 80], [(0, 7)], 0.1),  # a full 80-key block; 81 keys in two blocks (80 + 1)
    (2, 1, 130, 64, [130, 64], [(1, 5)], 0.0),  # key blocks
    (2, 2, 33, 128, [33, 16], None, 0.0),
    (2, 2, 24, 20, [24, 11], [(1, 5)], 0.0),  # head_dim not a multiple of 8
]
TERMS = [
    ("bias", dict(bias=True)),
    ("angle5", dict(bias=False, angle_rank=5)),
    ("message3", dict(bias=False, message_rank=3)),
    ("all16", dict(bias=True, angle_rank=16, message_rank=16)),
    ("all_r33_r64", dict(bias=True, angle_rank=33, message_rank=64)),
]


@pytest.mark.parametrize("terms", TERMS, ids=[t[0] for t in TERMS])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"B{s[0]}H{s[1]}N{s[2]}D{s[3]}")
def test_fp32_terms_match_fp64(cuda, shape, terms):
    B, H, N, D, counts, holes, drop = shape
    case = random_simplicial(B, H, N, D, seed=N + D + 7, counts=counts, holes=holes, pair_drop=drop,
                            std=logit_std(D))
    tm = make_terms(B, H, N, D, seed=N * 3 + D, **terms[1])
    out, lse, out32 = run(case, tm, cuda, torch.float32, "ieee_fp32")
    ref, ref_lse = oracle(case, tm, torch.float32)
    np.testing.assert_allclose(out32.cpu().numpy(), ref, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("terms", TERMS, ids=[t[0] for t in TERMS])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"B{s[0]}H{s[1]}N{s[2]}D{s[3]}")
def test_16bit_terms_match_fp64(cuda, shape, terms, dtype):
    B, H, N, D, counts, holes, drop = shape
    case = random_simplicial(B, H, N, D, seed=N + D + 8, counts=counts, holes=holes, pair_drop=drop,
                            std=logit_std(D))
    tm = make_terms(B, H, N, D, seed=N * 5 + D, **terms[1])
    out, lse, out32 = run(case, tm, cuda, dtype, "bf16_tc")
    ref, ref_lse = oracle(case, tm, dtype)
    assert out.dtype == dtype
    assert rel_err(out32.cpu().numpy(), ref) <= 2e-2
    assert rel_err(out.float().cpu().numpy(), ref) <= 2e-2
    worst = row_errors(out32.cpu().numpy(), ref, case[5]).max()
    print(f"worst row {worst:.3e}", flush=True)
    assert worst <= ROW_BAR
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=2e-2, atol=5e-2)


@pytest.mark.parametrize("shape", [(3, 2, 45, 64, [45, 30, 7], [(1, 2)], 0.1), (2, 1, 130, 64, [130, 77], None, 0.0)],
                         ids=["one_block", "key_blocks"])
def test_16bit_large_bias_takes_exact_offsets(cuda, shape):
    """Bias terms of several units in log2 units (beyond the one-pass bound and the shifted pass's cap): exact
    offsets (running maxima in one key block, two passes over key blocks), every valid query row against
    float64."""
    B, H, N, D, counts, holes, drop = shape
    case = random_simplicial(B, H, N, D, seed=N + 11, counts=counts, holes=holes, pair_drop=drop,
                            std=logit_std(D))
    tm = make_terms(B, H, N, D, seed=N + 12, scale=6.0)
    out, lse, out32 = run(case, tm, cuda, torch.bfloat16, "bf16_tc")
    ref, ref_lse = oracle(case, tm, torch.bfloat16)
    assert rel_err(out32.cpu().numpy(), ref) <= 2e-2
    worst = row_errors(out32.cpu().numpy(), ref, case[5]).max()
    print(f"worst row {worst:.3e}", flush=True)
    assert worst <= ROW_BAR
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=2e-2, atol=5e-2)


def test_16bit_masking_scale_bias(cuda):
    """A masking-style bias: u_ij = -1e4 on a random 30 % of (query, key) pairs, the rest N(0, 0.5^2), gates
    1 + N(0, 0.1^2).  c_i u_ij ~ -1.4e4 (log2 units) is staged as fp16 without saturating and drives those
    pairs' P to 0 exactly as exp(-1e4) does in float64; the exact offsets are taken over the rest.
    Bar: 2e-2 normwise and every valid row within the row bar of its norm."""
    B, H, N, D = 2, 2, 37, 64
    case = random_simplicial(B, H, N, D, seed=41, counts=[37, 23], std=logit_std(D))
    tm = make_terms(B, H, N, D, seed=42)
    gen = torch.Generator().manual_seed(43)
    u = tm["bias"][0]
    u[torch.rand(u.shape, generator=gen) < 0.3] = -1e4
    tm["bias"][3] = 1.0 + 0.1 * torch.randn(B, H, N, generator=gen)
    out, lse, out32 = run(case, tm, cuda, torch.bfloat16, "bf16_tc")
    ref, ref_lse = oracle(case, tm, torch.bfloat16)
    assert rel_err(out32.cpu().numpy(), ref) <= 2e-2
    worst = row_errors(out32.cpu().numpy(), ref, case[5]).max()
    print(f"masking-scale bias: worst row {worst:.3e}", flush=True)
    assert worst <= ROW_BAR


def test_16bit_dominant_pair_bias_near_fp16_limit(cuda):
    """One key pair per molecule made dominant by w_jk = 2e4 (gate 1: c w ~ 2.9e4 log2 units, below the fp16
    limit of 65504 the staged products saturate at): every valid query's output is v1_j (.) v2_k of that pair,
    as in float64.  Bar: 2e-2 normwise and the row bar per valid row."""
    B, H, N, D = 2, 2, 29, 64
    case = random_simplicial(B, H, N, D, seed=44, counts=[29, 17], std=logit_std(D))
    tm = make_terms(B, H, N, D, seed=45)
    tm["bias"][2][0, :, 3, 5] = 2e4
    tm["bias"][2][1, :, 11, 2] = 2e4
    tm["bias"][3] = torch.ones(B, H, N)
    out, lse, out32 = run(case, tm, cuda, torch.bfloat16, "bf16_tc")
    ref, ref_lse = oracle(case, tm, torch.bfloat16)
    assert rel_err(out32.cpu().numpy(), ref) <= 2e-2
    worst = row_errors(out32.cpu().numpy(), ref, case[5]).max()
    print(f"dominant pair bias: worst row {worst:.3e}", flush=True)
    assert worst <= ROW_BAR


def _small_logit_case(B, H, N, D, seed, counts):
    """q scaled by 0.05, so that the logit bound of a query is about 4.5 log2 units and the bias decides
    whether a unit stays within the one-pass bound (13.5), takes the shifted one pass (bound <= 24) or
    neither."""
    case = list(random_simplicial(B, H, N, D, seed=seed, counts=counts, std=logit_std(D)))
    case[0] = case[0] * 0.05
    return tuple(case)


def test_16bit_shifted_one_pass_matches_fp64(cuda):
    """Bias N(0, 0.5^2), gates N(0, 1): queries with large gates put their units past the one-pass bound but
    below the shifted pass's cap; the shifted pass (offset max(B_i - 14, 0) per query) keeps them.  Every
    valid query row against float64, and the lse, which carries each query's offset."""
    B, H, N, D = 3, 4, 45, 64
    case = _small_logit_case(B, H, N, D, 47, [45, 33, 12])
    tm = make_terms(B, H, N, D, seed=48)
    out, lse, out32 = run(case, tm, cuda, torch.bfloat16, "bf16_tc")
    ref, ref_lse = oracle(case, tm, torch.bfloat16)
    assert rel_err(out32.cpu().numpy(), ref) <= 2e-2
    worst = row_errors(out32.cpu().numpy(), ref, case[5]).max()
    print(f"shifted one pass: worst row {worst:.3e}", flush=True)
    assert worst <= ROW_BAR
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=2e-2, atol=5e-2)


def test_16bit_shifted_pass_falls_back_when_its_denominators_underflow(cuda):
    """u = -10 on every pair, v = w = 0, gate 1: c u = -14.4 log2 units, so each query's bound (~19) is past
    the one-pass bound and below the shifted pass's cap, but the bound's offset leaves every 2^(S - m_i) near
    2^-19: the denominators stay far below the pass's floor and the unit reruns with exact offsets.  The
    constant cancels in the softmax; output and lse against float64."""
    B, H, N, D = 2, 2, 41, 64
    case = _small_logit_case(B, H, N, D, 46, [41, 26])
    tm = {"bias": [torch.full((B, H, N, N), -10.0), torch.zeros(B, H, N, N), torch.zeros(B, H, N, N),
                   torch.ones(B, H, N)]}
    out, lse, out32 = run(case, tm, cuda, torch.bfloat16, "bf16_tc")
    ref, ref_lse = oracle(case, tm, torch.bfloat16)
    assert rel_err(out32.cpu().numpy(), ref) <= 2e-2
    worst = row_errors(out32.cpu().numpy(), ref, case[5]).max()
    print(f"shifted pass fallback: worst row {worst:.3e}", flush=True)
    assert worst <= ROW_BAR
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=2e-2, atol=5e-2)


def test_fp32_bias_with_bf16_operands(cuda):
    """The module passes the bias in its own dtype: fp32 bias with bf16 operands."""
    case = random_simplicial(2, 2, 40, 64, seed=3, counts=[40, 21], std=logit_std(64))
    tm = make_terms(2, 2, 40, 64, seed=4)
    out, lse, out32 = run(case, tm, cuda, torch.bfloat16, "bf16_tc", bias_dtype=torch.float32)
    ref, ref_lse = oracle(case, tm, torch.bfloat16, bias_dtype=torch.float32)
    assert rel_err(out32.cpu().numpy(), ref) <= 2e-2


def test_zero_gate_bias_equals_no_bias(cuda):
    """gate = 0 removes the bias exactly (u, v, w enter only through gate * (.))."""
    case = random_simplicial(2, 2, 37, 64, seed=5, counts=[37, 20], std=logit_std(64))
    tm = make_terms(2, 2, 37, 64, seed=6)
    tm["bias"][3] = torch.zeros_like(tm["bias"][3])
    with_bias = run(case, tm, cuda, torch.float32, "ieee_fp32")[2]
    plain = run(case, {}, cuda, torch.float32, "ieee_fp32")[2]
    np.testing.assert_allclose(with_bias.cpu().numpy(), plain.cpu().numpy(), rtol=1e-5, atol=1e-6)


def test_qm9_config_with_bias_whole_batch(cuda):
    """Config 1 (fp32, 128 molecules) with a factorized bias, every molecule against float64."""
    w = simplicial_workload("qm9")
    B, H, N, D = w.shape
    case = (w.q, w.k1, w.v1, w.k2, w.v2, w.query_valid, w.pair_key_valid, None)
    tm = make_terms(B, H, N, D, seed=101)
    out, lse, out32 = run(case, tm, cuda, torch.float32, "ieee_fp32")
    ref, ref_lse = oracle(case, tm, torch.float32)
    np.testing.assert_allclose(out32.cpu().numpy(), ref, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=1e-4, atol=1e-4)


def test_geom_config_with_bias_whole_batch(cuda):
    """Config 2 (bf16, 64 molecules up to 181 atoms) with a factorized bias, every molecule against float64."""
    w = simplicial_workload("geom")
    B, H, N, D = w.shape
    case = (w.q, w.k1, w.v1, w.k2, w.v2, w.query_valid, w.pair_key_valid, None)
    tm = make_terms(B, H, N, D, seed=102)
    out, lse, out32 = run(case, tm, cuda, torch.bfloat16, "bf16_tc")
    ref, ref_lse = oracle(case, tm, torch.bfloat16)
    assert rel_err(out32.cpu().numpy(), ref) <= 2e-2
    worst = row_errors(out32.cpu().numpy(), ref, w.query_valid).max()
    print(f"config 2 with bias: worst row {worst:.3e}", flush=True)
    assert worst <= ROW_BAR
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=2e-2, atol=5e-2)


def test_module_auto_dispatch_serves_factorized_bias_on_gpu(cuda):
    """The default trunk's call (factorized bias, bf16_tc) runs the HIP kernel under impl="auto" and
    agrees with the torch path of the same module."""
    torch.manual_seed(0)
    attn = SimplicialAttention(dim=64, num_heads=4, impl="auto", precision="bf16_tc").to(cuda)
    x = torch.randn(3, 19, 64, device=cuda)
    kpm = torch.zeros(3, 19, dtype=torch.bool, device=cuda)
    kpm[1, 12:] = True
    kpm[2, 5:] = True
    fb = SimplicialFactorizedBias(*(torch.randn(3, 4, 19, 19, device=cuda) * 0.5 for _ in range(3)),
                                  gate=torch.randn(3, 4, 19, device=cuda))
    got = attn(x, key_padding_mask=kpm, factorized_bias=fb)
    assert attn._last_impl_used == "triton"
    attn.impl = "torch"
    ref = attn(x, key_padding_mask=kpm, factorized_bias=fb)
    assert attn._last_impl_used == "torch"
    assert rel_err(got.detach().cpu().numpy(), ref.detach().cpu().double().numpy()) <= 2e-2


def test_module_all_terms_fp32_matches_torch_path(cuda):
    """impl="triton" with every optional term (angle and message cast to fp32 as the reference does)."""
    torch.manual_seed(1)
    attn = SimplicialAttention(dim=32, num_heads=2, impl="triton", precision="ieee_fp32", message_mode="low_rank",
                               message_rank=4).to(cuda)
    B, T = 2, 9
    x = torch.randn(B, T, 32, device=cuda)
    mask = SimplicialAttentionMask(query_valid=torch.ones(B, T, dtype=torch.bool, device=cuda),
                                   pair_key_valid=torch.ones(B, T, dtype=torch.bool, device=cuda),
                                   pair_valid=torch.rand(B, T, T, device=cuda) > 0.2)
    fb = SimplicialFactorizedBias(*(torch.randn(B, 2, T, T, device=cuda) for _ in range(3)),
                                  gate=torch.randn(B, 2, T, device=cuda))
    ar = SimplicialLowRankAngleResidual(left=torch.randn(B, 2, T, T, 3, device=cuda),
                                        right=torch.randn(B, 2, T, T, 3, device=cuda),
                                        gate=torch.randn(B, 2, T, device=cuda))
    mr = SimplicialLowRankMessageResidual(left=torch.randn(B, 2, T, T, 4, device=cuda),
                                          right=torch.randn(B, 2, T, T, 4, device=cuda))
    got = attn(x, attention_mask=mask, factorized_bias=fb, angle_residual=ar, message_residual=mr)
    assert attn._last_impl_used == "triton"
    q, k1, v1, k2, v2 = attn._project_inputs(x)
    heads = simplicial_attention_torch_from_projected(
        q, k1, v1, k2, v2, attention_mask=mask, factorized_bias=fb, angle_residual=ar, message_residual=mr,
        message_basis=attn.message_basis, fp32_core=True)
    ref = attn.out_proj(attn._merge_heads(heads))
    torch.testing.assert_close(got, ref, rtol=1e-4, atol=1e-4)


def test_launcher_rejects_mismatched_terms(cuda):
    case = random_simplicial(1, 2, 8, 16, seed=1)
    q, k1, v1, k2, v2, qv, pkv = (t.to(cuda) for t in case[:7])
    bad = torch.randn(1, 2, 8, 7, device=cuda)
    with pytest.raises(ValueError, match="must have shape"):
        hip_simplicial_attention_forward(q, k1, v1, k2, v2, query_valid=qv, pair_key_valid=pkv, pair_valid=None,
                                         u=bad, v_bias=bad, w=bad, gate=torch.randn(1, 2, 8, device=cuda))
    left = torch.randn(1, 2, 8, 8, 3, device=cuda)
    with pytest.raises(ValueError, match="same shape"):
        hip_simplicial_attention_forward(q, k1, v1, k2, v2, query_valid=qv, pair_key_valid=pkv, pair_valid=None,
                                         angle_left=left, angle_right=left[..., :2],
                                         angle_gate=torch.randn(1, 2, 8, device=cuda))
    with pytest.raises(ValueError, match="message_basis must have shape"):
        hip_simplicial_attention_forward(q, k1, v1, k2, v2, query_valid=qv, pair_key_valid=pkv, pair_valid=None,
                                         message_left=left, message_right=left,
                                         message_basis=torch.randn(2, 4, 16, device=cuda))
