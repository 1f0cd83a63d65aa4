"""GPU parity of the HIP 2-simplicial forward (mf_simplicial_fwd) against the CPU oracle.

Tolerances: fp32 operands <= 1e-4 (the reference's
own GPU parity bar, tests/test_simplicial_attention.py:886), 16-bit operands
normwise relative error <= 2e-2 against the float64 result on the same
16-bit-rounded inputs.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from matterformer_amd import _native
from matterformer_amd.hip_simplicial_attention import hip_simplicial_attention_forward
from matterformer_amd.workloads import random_simplicial, simplicial_workload
from oracle.simplicial import brute_force_fp64, reference_path

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def run_hip(case, device, dtype, precision="bf16_tc", need_state=True):
    q, k1, v1, k2, v2, qv, pkv, pv = case
    ops = [t.to(dtype).to(device) for t in (q, k1, v1, k2, v2)]
    out, lse, out32 = hip_simplicial_attention_forward(
        *ops, query_valid=qv.to(device), pair_key_valid=pkv.to(device),
        pair_valid=None if pv is None else pv.to(device), precision=precision, need_backward_state=need_state)
    torch.cuda.synchronize()
    return out, lse, out32


def oracle64(case, dtype):
    q, k1, v1, k2, v2, qv, pkv, pv = case
    ops = [t.to(dtype).double().numpy() for t in (q, k1, v1, k2, v2)]
    return brute_force_fp64(*ops, qv.numpy(), pkv.numpy(), None if pv is None else pv.numpy())


def logit_std(D):
    # per-element std giving logits S = sum_d q k1 k2 a standard deviation of ~2
    return (4.0 / D) ** (1.0 / 6.0)


def rel_err(got, ref):
    got = np.asarray(got, dtype=np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


SHAPES = [
    # (B, H, N, D, counts, holes, pair_drop)
    (2, 4, 5, 8, [4, 2], None, 0.0),          # the reference's parity-test shape
    (1, 2, 7, 8, [5], None, 0.3),             # pair_valid (reference all-features shape)
    (3, 2, 29, 32, [29, 17, 9], [(0, 3)], 0.0),
    (2, 2, 70, 64, [70, 41], None, 0.0),      # two key chunks
    (2, 1, 130, 64, [130, 64], None, 0.1),    # three key chunks + pair mask
    (2, 2, 33, 128, [33, 16], None, 0.0),
    (2, 2, 24, 20, [24, 11], [(1, 5)], 0.0),  # head_dim not a multiple of 8
    (2, 2, 16, 64, [16, 1], None, 0.0),       # single-atom molecule
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"B{s[0]}H{s[1]}N{s[2]}D{s[3]}")
def test_fp32_matches_fp64_oracle(cuda, shape):
    B, H, N, D, counts, holes, drop = shape
    case = random_simplicial(B, H, N, D, seed=N + D, counts=counts, holes=holes, pair_drop=drop,
                            std=logit_std(D))
    out, lse, out32 = run_hip(case, cuda, torch.float32, precision="ieee_fp32")
    ref, ref_lse = oracle64(case, torch.float32)
    np.testing.assert_allclose(out32.cpu().numpy(), ref, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"B{s[0]}H{s[1]}N{s[2]}D{s[3]}")
def test_16bit_matches_fp64_oracle(cuda, shape, dtype):
    B, H, N, D, counts, holes, drop = shape
    case = random_simplicial(B, H, N, D, seed=N + D + 1, counts=counts, holes=holes, pair_drop=drop,
                            std=logit_std(D))
    out, lse, out32 = run_hip(case, cuda, dtype)
    ref, ref_lse = oracle64(case, dtype)
    assert out.dtype == dtype
    assert rel_err(out32.cpu().numpy(), ref) <= 2e-2
    assert rel_err(out.float().cpu().numpy(), ref) <= 2e-2
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=2e-2, atol=5e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("D, qscale", [(64, 0.2), (32, 0.3)], ids=["D64", "D32"])
def test_16bit_shifted_one_pass_matches_fp64(cuda, dtype, D, qscale):
    """q scaled so that each query's logit bound sum_d |q_d| max|k1_d| max|k2_d| is about 18 log2 units:
    past the one-pass bound (13.5) and within the shifted pass's cap (24), whose per-query offset
    max(bound - 14, 0) keeps every 2^(S - m) below 2^14.  Output and lse (which carries the offset)
    against float64."""
    case = list(random_simplicial(3, 2, 41, D, seed=D + 5, counts=[41, 30, 9], std=logit_std(D)))
    case[0] = case[0] * qscale
    out, lse, out32 = run_hip(tuple(case), cuda, dtype)
    ref, ref_lse = oracle64(tuple(case), dtype)
    assert rel_err(out32.cpu().numpy(), ref) <= 2e-2
    assert rel_err(out.float().cpu().numpy(), ref) <= 2e-2
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=2e-2, atol=5e-2)


def test_16bit_ieee_precision_upcasts(cuda):
    case = random_simplicial(2, 2, 21, 16, seed=3, counts=[21, 8])
    out, lse, out32 = run_hip(case, cuda, torch.bfloat16, precision="ieee_fp32")
    ref, ref_lse = oracle64(case, torch.bfloat16)
    np.testing.assert_allclose(out32.cpu().numpy(), ref, rtol=1e-4, atol=1e-4)
    assert out.dtype == torch.bfloat16


@pytest.mark.parametrize("name", ["fp32_padding", "fp32_holes_pairvalid", "fp32_qm9_slice",
                                  "bf16_native", "bf16_fp32core", "bf16_geom_slice"])
def test_reference_golden_vectors(cuda, name):
    z = np.load(GOLDEN / f"simplicial_{name}.npz")
    dtype = getattr(torch, str(z["dtype"]))
    ops = [torch.from_numpy(z[k]) for k in ("q", "k1", "v1", "k2", "v2")]
    qv, pkv = torch.from_numpy(z["query_valid"]), torch.from_numpy(z["pair_key_valid"])
    pv = torch.from_numpy(z["pair_valid"]) if "pair_valid" in z.files else None
    out, _, out32 = run_hip((*ops, qv, pkv, pv), cuda, dtype, precision="bf16_tc" if dtype != torch.float32 else "ieee_fp32")
    expected = z["out"].astype(np.float64)
    if dtype == torch.float32:
        np.testing.assert_allclose(out32.cpu().numpy(), expected, rtol=1e-4, atol=1e-4)
    else:
        assert rel_err(out.float().cpu().numpy(), expected) <= 2e-2


def test_single_valid_pair_kat(cuda):
    q = torch.zeros(1, 1, 3, 2)
    v1 = torch.tensor([[[[1.0, 2.0], [5.0, 7.0], [11.0, 13.0]]]])
    v2 = torch.tensor([[[[3.0, 5.0], [17.0, 19.0], [23.0, 29.0]]]])
    pv = torch.zeros(1, 3, 3, dtype=torch.bool)
    pv[:, 0, 0] = True
    valid = torch.ones(1, 3, dtype=torch.bool)
    out, lse, _ = run_hip((q, q.clone(), v1, q.clone(), v2, valid, valid, pv), cuda, torch.float32, "ieee_fp32")
    assert torch.allclose(out.cpu(), torch.tensor([3.0, 10.0]).expand(1, 1, 3, 2), atol=1e-6)
    assert torch.allclose(lse.cpu(), torch.zeros(1, 1, 3), atol=1e-6)


def test_empty_rows_are_zero(cuda):
    # molecule 0: no valid keys but valid queries; molecule 1: nothing valid;
    # molecule 2: keys valid but every pair masked.
    B, H, N, D = 3, 2, 12, 16
    case = list(random_simplicial(B, H, N, D, seed=7))
    qv = torch.ones(B, N, dtype=torch.bool)
    pkv = torch.ones(B, N, dtype=torch.bool)
    pkv[0] = False
    qv[1] = False
    pkv[1] = False
    pv = torch.ones(B, N, N, dtype=torch.bool)
    pv[2] = False
    case[5:8] = [qv, pkv, pv]
    out, lse, out32 = run_hip(tuple(case), cuda, torch.bfloat16)
    assert torch.count_nonzero(out) == 0 and torch.count_nonzero(out32) == 0 and torch.count_nonzero(lse) == 0


def test_inference_mode_matches_training_outputs(cuda):
    case = random_simplicial(4, 3, 37, 64, seed=11, counts=[37, 20, 5, 30])
    a, _, _ = run_hip(case, cuda, torch.bfloat16, need_state=True)
    b, lse, o32 = run_hip(case, cuda, torch.bfloat16, need_state=False)
    assert lse is None and o32 is None
    assert torch.equal(a, b)


def test_deterministic(cuda):
    case = random_simplicial(3, 2, 50, 64, seed=12, counts=[50, 31, 44])
    a = run_hip(case, cuda, torch.bfloat16)[2]
    b = run_hip(case, cuda, torch.bfloat16)[2]
    assert torch.equal(a, b)


def test_geom_config_full_size(cuda):
    """Config 2 at full size: finite, zero padded rows, per-molecule parity on a sample,
    and batch invariance (a molecule alone gives the same bits as inside the batch)."""
    w = simplicial_workload("geom")
    wd = w.to(cuda, torch.bfloat16)
    out, lse, out32 = hip_simplicial_attention_forward(
        wd.q, wd.k1, wd.v1, wd.k2, wd.v2, query_valid=wd.query_valid, pair_key_valid=wd.pair_key_valid,
        pair_valid=None, precision="bf16_tc")
    torch.cuda.synchronize()
    assert torch.isfinite(out32).all()
    pad = ~w.query_valid
    assert torch.count_nonzero(out32.cpu().permute(0, 2, 1, 3)[pad]) == 0
    sample = [int(torch.argmax(w.counts)), int(torch.argmin(w.counts)), 0, 17]
    for b in sample:
        n = int(w.counts[b])
        sl = [t[b:b + 1, :, :n].to(torch.bfloat16) for t in (w.q, w.k1, w.v1, w.k2, w.v2)]
        ones = torch.ones(1, n, dtype=torch.bool)
        ref, ref_lse = brute_force_fp64(*(t.double().numpy() for t in sl), ones.numpy(), ones.numpy())
        got = out32[b:b + 1, :, :n].cpu().numpy()
        assert rel_err(got, ref) <= 2e-2, b
        np.testing.assert_allclose(lse[b:b + 1, :, :n].cpu().numpy(), ref_lse, rtol=2e-2, atol=5e-2)
        alone = hip_simplicial_attention_forward(
            *(t[b:b + 1] for t in (wd.q, wd.k1, wd.v1, wd.k2, wd.v2)), query_valid=wd.query_valid[b:b + 1],
            pair_key_valid=wd.pair_key_valid[b:b + 1], pair_valid=None, precision="bf16_tc")[2]
        assert torch.equal(alone, out32[b:b + 1]), b


def test_qm9_config_matches_reference_cpu_path(cuda):
    """Config 1 (fp32): HIP fp32 path vs the oracle's torch-CPU reference path."""
    w = simplicial_workload("qm9")
    ref = reference_path(w.q, w.k1, w.v1, w.k2, w.v2, w.query_valid, w.pair_key_valid, chunk_size=128)
    wd = w.to(cuda)
    out, _, _ = hip_simplicial_attention_forward(
        wd.q, wd.k1, wd.v1, wd.k2, wd.v2, query_valid=wd.query_valid, pair_key_valid=wd.pair_key_valid,
        pair_valid=None, precision="ieee_fp32")
    np.testing.assert_allclose(out.cpu().numpy(), ref.numpy(), rtol=1e-4, atol=1e-4)


def test_library_reports_unsupported_shape(cuda):
    lib = _native.lib()
    assert lib.mf_simplicial_fwd_supported(64, 8, 181, 64, _native.MF_DTYPE_BF16) == _native.MF_OK
    assert lib.mf_simplicial_fwd_supported(1, 1, 8, 256, _native.MF_DTYPE_BF16) == _native.MF_ERR_UNSUPPORTED
    assert "head_dim" in _native.last_error()
