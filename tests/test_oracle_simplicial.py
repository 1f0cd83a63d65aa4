"""Pins the CPU oracle of 2-simplicial attention (oracle/simplicial.py).

* against golden vectors written from the reference itself (tests/golden/);
* ``reference_path`` against the independent float64 brute force;
* both against closed forms and the reference's KATs
  (tests/test_simplicial_attention.py:415-463 of stases/Matterformer).
"""

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.simplicial import brute_force_fp64, reference_path, work_flops
from matterformer_amd.workloads import random_simplicial, simplicial_workload

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = sorted(p.stem for p in GOLDEN.glob("simplicial_*.npz"))


def load_case(name):
    z = np.load(GOLDEN / f"{name}.npz")
    dtype = getattr(torch, str(z["dtype"]))
    t = {k: torch.from_numpy(z[k]) for k in z.files if z[k].dtype != np.dtype("<U0") and z[k].ndim > 0}
    ops = [t[k].to(dtype) for k in ("q", "k1", "v1", "k2", "v2")]
    opt = {}
    if "u" in t:
        opt["factorized_bias"] = tuple(t[k].to(dtype) for k in ("u", "v_bias", "w", "gate"))
    if "angle_left" in t:
        opt["angle_residual"] = tuple(t[k].to(dtype) for k in ("angle_left", "angle_right", "angle_gate"))
    if "message_left" in t:
        opt["message_residual"] = tuple(t[k].to(dtype) for k in ("message_left", "message_right", "message_basis"))
    return z, ops, t["query_valid"], t["pair_key_valid"], t.get("pair_valid"), opt


@pytest.mark.parametrize("name", CASES)
def test_reference_path_reproduces_reference_golden_vectors(name):
    z, ops, qv, pkv, pv, opt = load_case(name)
    out = reference_path(*ops, qv, pkv, pv, chunk_size=int(z["chunk_size"]), fp32_core=bool(z["fp32_core"]), **opt)
    expected = torch.from_numpy(z["out"])
    # Same ATen operations in the same order: bit-identical.
    assert torch.equal(out.float(), expected), (out.float() - expected).abs().max()


@pytest.mark.parametrize("name", [c for c in CASES if "bias" not in c])
def test_golden_vectors_agree_with_fp64_brute_force(name):
    z, ops, qv, pkv, pv, _ = load_case(name)
    ref, _ = brute_force_fp64(*(o.float().numpy() for o in ops), qv.numpy(), pkv.numpy(),
                              None if pv is None else pv.numpy())
    got = z["out"].astype(np.float64)
    tol = 1e-5 if str(z["out_dtype"]) == "float32" else 2e-2
    err = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert err <= tol, err


def test_brute_force_optional_terms_match_reference_golden():
    """The reference's own bias + angle + message fixture pins each optional term of the brute force;
    dropping any one of them (or transposing u and v) moves the result far outside the tolerance."""
    z, ops, qv, pkv, pv, opt = load_case("simplicial_fp32_bias_angle_message")
    args = [o.numpy() for o in ops] + [qv.numpy(), pkv.numpy(), pv.numpy()]
    terms = dict(bias=tuple(a.numpy() for a in opt["factorized_bias"]),
                 angle=tuple(a.numpy() for a in opt["angle_residual"]),
                 message=tuple(a.numpy() for a in opt["message_residual"]))
    expected = z["out"].astype(np.float64)
    ref, _ = brute_force_fp64(*args, **terms)
    np.testing.assert_allclose(ref, expected, rtol=1e-5, atol=1e-5)
    for drop in terms:
        partial = {k: v for k, v in terms.items() if k != drop}
        bad, _ = brute_force_fp64(*args, **partial)
        assert np.abs(bad - expected).max() > 1e-2, drop
    u, v, w, g = terms["bias"]
    bad, _ = brute_force_fp64(*args, **{**terms, "bias": (v, u, w, g)})
    assert np.abs(bad - expected).max() > 1e-2


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_reference_path_matches_brute_force_fp32(seed):
    q, k1, v1, k2, v2, qv, pkv, pv = random_simplicial(3, 2, 11, 8, seed=seed, counts=[11, 7, 3],
                                                       holes=[(0, 2)], pair_drop=0.25 * seed)
    out = reference_path(q, k1, v1, k2, v2, qv, pkv, pv, chunk_size=4)
    ref, _ = brute_force_fp64(q.numpy(), k1.numpy(), v1.numpy(), k2.numpy(), v2.numpy(), qv.numpy(), pkv.numpy(),
                              None if pv is None else pv.numpy())
    np.testing.assert_allclose(out.numpy(), ref, rtol=1e-5, atol=1e-6)


def test_single_valid_pair_kat():
    # tests/test_simplicial_attention.py:448-463: only pair (0,0) valid -> v1_0 (.) v2_0 = [3, 10]
    q = np.zeros((1, 1, 3, 2))
    k1 = np.zeros((1, 1, 3, 2))
    v1 = np.array([[[[1.0, 2.0], [5.0, 7.0], [11.0, 13.0]]]])
    k2 = np.zeros((1, 1, 3, 2))
    v2 = np.array([[[[3.0, 5.0], [17.0, 19.0], [23.0, 29.0]]]])
    pv = np.zeros((1, 3, 3), dtype=bool)
    pv[:, 0, 0] = True
    qv = np.ones((1, 3), dtype=bool)
    out, lse = brute_force_fp64(q, k1, v1, k2, v2, qv, qv, pv)
    np.testing.assert_allclose(out, np.broadcast_to([3.0, 10.0], out.shape))
    np.testing.assert_allclose(lse, 0.0)
    t = [torch.from_numpy(a).float() for a in (q, k1, v1, k2, v2)]
    out_t = reference_path(*t, torch.from_numpy(qv), torch.from_numpy(qv), torch.from_numpy(pv), chunk_size=3)
    np.testing.assert_allclose(out_t.numpy(), out, atol=1e-6)


def test_zero_query_closed_form_and_lse():
    # q = 0 -> uniform over valid pairs: out = mean_j v1_j (.) mean_k v2_k, lse = log(n^2)
    q, k1, v1, k2, v2, qv, pkv, _ = random_simplicial(2, 3, 9, 5, seed=5, counts=[9, 4])
    q = torch.zeros_like(q)
    out, lse = brute_force_fp64(q.numpy(), k1.numpy(), v1.numpy(), k2.numpy(), v2.numpy(), qv.numpy(), pkv.numpy())
    for b, n in enumerate([9, 4]):
        want = v1[b, :, :n].double().mean(1) * v2[b, :, :n].double().mean(1)
        np.testing.assert_allclose(out[b, :, :n], want[:, None, :].expand(-1, n, -1).numpy(), rtol=1e-12)
        np.testing.assert_allclose(lse[b, :, :n], math.log(n * n), rtol=1e-12)
        assert np.all(out[b, :, n:] == 0) and np.all(lse[b, :, n:] == 0)
    out_t = reference_path(q, k1, v1, k2, v2, qv, pkv, chunk_size=128)
    np.testing.assert_allclose(out_t.numpy(), out, rtol=1e-5, atol=1e-6)


def test_masked_keys_do_not_change_output():
    # tests/test_simplicial_attention.py:415-445
    torch.manual_seed(0)
    q, k1, v1, k2, v2 = (torch.randn(1, 1, 3, 4) for _ in range(5))
    qv = torch.tensor([[True, True, True]])
    pkv = torch.tensor([[True, True, False]])
    out = reference_path(q, k1, v1, k2, v2, qv, pkv, chunk_size=3)
    k1a, v1a, k2a, v2a = (t.clone() for t in (k1, v1, k2, v2))
    k1a[..., 2, :], v1a[..., 2, :], k2a[..., 2, :], v2a[..., 2, :] = 1e3, -1e3, 2e3, 3e3
    out_alt = reference_path(q, k1a, v1a, k2a, v2a, qv, pkv, chunk_size=3)
    assert torch.allclose(out, out_alt, atol=1e-6, rtol=1e-5)
    ref, _ = brute_force_fp64(q.numpy(), k1a.numpy(), v1a.numpy(), k2a.numpy(), v2a.numpy(), qv.numpy(), pkv.numpy())
    np.testing.assert_allclose(out.numpy(), ref, rtol=1e-5, atol=1e-6)


def test_brute_force_catches_transposed_operands():
    # A planted mistake (k1 and k2 swapped) must be visible to the oracle comparison.
    q, k1, v1, k2, v2, qv, pkv, _ = random_simplicial(1, 2, 6, 4, seed=9, std=1.0)
    good, _ = brute_force_fp64(q.numpy(), k1.numpy(), v1.numpy(), k2.numpy(), v2.numpy(), qv.numpy(), pkv.numpy())
    bad, _ = brute_force_fp64(q.numpy(), k2.numpy(), v1.numpy(), k1.numpy(), v2.numpy(), qv.numpy(), pkv.numpy())
    assert np.abs(good - bad).max() > 1e-3


def test_workload_generators_follow_baseline_configs():
    w = simplicial_workload("geom")
    assert w.shape == (64, 8, 181, 64)
    assert int(w.counts.min()) >= 10 and int(w.counts.max()) <= 181
    assert abs(float(w.counts.float().mean()) - 44.0) < 6.0
    assert work_flops(w.pair_key_valid.numpy(), w.query_valid.numpy(), 8, 64) == w.valid_flops()
    w1 = simplicial_workload("qm9")
    assert w1.shape == (128, 8, 29, 32)
    assert int(w1.counts.min()) >= 9 and int(w1.counts.max()) <= 29
    again = simplicial_workload("geom")
    assert torch.equal(again.q, w.q) and torch.equal(again.counts, w.counts)
