"""GPU parity of the 16-bit pair kernel behind mf_simplicial_fwd (bf16/fp16, head_dim <= 64).

The kernel stages each (molecule, head) as fp16 scaled by powers of two and
picks, per unit, between P = 2^S directly (when the a-priori bound on |S| is
at most 13.5 and the query scale needs no rescaling) and a two-pass
exact-maximum mode; inputs are scaled here so that each mode is exercised:
std 0.05 keeps every logit bound small, std 1.3 pushes the bound past the
limit, and the extreme-scale case forces the rescaled two-pass mode.
Molecules with more than 128 keys are taken in key blocks (the mixed-size
cases), molecules with more than 48 queries in several query groups.
Tolerance: normwise relative error <= 2e-2 against the float64 oracle on the
same 16-bit-rounded inputs.
"""

import numpy as np
import pytest
import torch

from matterformer_amd.hip_simplicial_attention import hip_simplicial_attention_forward
from matterformer_amd.workloads import random_simplicial
from oracle.simplicial import brute_force_fp64

pytestmark = pytest.mark.gpu


def run(case, device, dtype):
    q, k1, v1, k2, v2, qv, pkv, pv = case
    ops = [t.to(dtype).to(device) for t in (q, k1, v1, k2, v2)]
    out, lse, out32 = hip_simplicial_attention_forward(
        *ops, query_valid=qv.to(device), pair_key_valid=pkv.to(device),
        pair_valid=None if pv is None else pv.to(device), precision="bf16_tc")
    torch.cuda.synchronize()
    ref, ref_lse = brute_force_fp64(*(t.to(dtype).double().numpy() for t in (q, k1, v1, k2, v2)), qv.numpy(),
                                    pkv.numpy(), None if pv is None else pv.numpy())
    return out, lse, out32, ref, ref_lse


def rel(got, ref):
    got = np.asarray(got, dtype=np.float64)
    return float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))


CASES = [
    # (B, H, N, D, counts, holes, pair_drop)
    (2, 4, 5, 8, [4, 2], None, 0.0),
    (3, 2, 29, 32, [29, 17, 9], [(0, 3)], 0.0),
    (2, 2, 80, 64, [80, 47], None, 0.0),          # full capacity, 5 key tiles
    (3, 2, 64, 64, [64, 33, 16], [(1, 2)], 0.2),  # pair_valid
    (2, 3, 96, 32, [96, 65], None, 0.0),          # head_dim 32 capacity (6 tiles)
    (2, 2, 24, 20, [24, 11], [(1, 5)], 0.0),      # head_dim not a multiple of 8
    (4, 1, 17, 64, [17, 1, 16, 3], None, 0.0),    # 1-atom molecule, odd tile counts
]


@pytest.mark.parametrize("std", [0.05, 1.3], ids=["bound", "twopass"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("shape", CASES, ids=lambda s: f"B{s[0]}H{s[1]}N{s[2]}D{s[3]}")
def test_fast_path_matches_oracle(cuda, shape, dtype, std):
    B, H, N, D, counts, holes, drop = shape
    case = random_simplicial(B, H, N, D, seed=N * D + B, counts=counts, holes=holes, pair_drop=drop, std=std)
    out, lse, out32, ref, ref_lse = run(case, cuda, dtype)
    assert torch.isfinite(out32).all()
    assert rel(out32.cpu().numpy(), ref) <= 2e-2
    assert rel(out.float().cpu().numpy(), ref) <= 2e-2
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=2e-2, atol=5e-2)
    qv = case[5]
    assert torch.count_nonzero(out32.cpu().permute(0, 2, 1, 3)[~qv]) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_mixed_sizes_fast_and_general(cuda, dtype):
    # molecules on both sides of the 128-key block in one call
    B, H, N, D = 4, 2, 150, 64
    case = random_simplicial(B, H, N, D, seed=5, counts=[150, 80, 81, 12], holes=[(0, 7)], std=0.08)
    out, lse, out32, ref, ref_lse = run(case, cuda, dtype)
    for b in range(B):
        assert rel(out32[b].cpu().numpy(), ref[b]) <= 2e-2, b
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=2e-2, atol=5e-2)


def test_large_batch_is_chunked(cuda):
    # more molecules than one launch takes (256 per launch)
    B, H, N, D = 1100, 1, 8, 8
    gen = torch.Generator().manual_seed(3)
    counts = torch.randint(1, N + 1, (B,), generator=gen).tolist()
    case = random_simplicial(B, H, N, D, seed=4, counts=counts, std=0.5)
    out, lse, out32, ref, ref_lse = run(case, cuda, torch.bfloat16)
    assert rel(out32.cpu().numpy(), ref) <= 2e-2
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=2e-2, atol=5e-2)


def test_scaled_inputs_give_same_softmax(cuda):
    # Scaling q changes which softmax mode runs but not the math: both results
    # must match their own oracle, and the bound mode must agree with the
    # two-pass mode on an input where both are exact (q scaled by a power of two
    # keeps bf16 products exact up to the exponent).
    B, H, N, D = 2, 2, 40, 64
    case = list(random_simplicial(B, H, N, D, seed=8, counts=[40, 23], std=0.7))
    for scale in (0.25, 8.0):
        c = list(case)
        c[0] = case[0] * scale
        out, lse, out32, ref, ref_lse = run(tuple(c), cuda, torch.bfloat16)
        assert rel(out32.cpu().numpy(), ref) <= 2e-2, scale
        np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=2e-2, atol=5e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_extreme_scale_rescaled_two_pass(cuda, dtype):
    # Large components in different head dimensions of q (d = 0), k1 (d = 1)
    # and k2 (d = 2): max|q log2 e| max|k1| max|k2| is far beyond what the
    # fp16 query operand can carry at the scale that keeps S in log2 units,
    # so the unit rescales S in the two-pass mode, while every product
    # q_d k1_d k2_d, and so every logit, stays moderate
    B, H, N, D = 2, 2, 33, 64
    case = list(random_simplicial(B, H, N, D, seed=11, counts=[33, 20], std=0.1))
    case[0][..., 0] += 100.0
    case[1][..., 1] += 50.0
    case[3][..., 2] += 50.0
    out, lse, out32, ref, ref_lse = run(tuple(case), cuda, dtype)
    assert torch.isfinite(out32).all()
    assert rel(out32.cpu().numpy(), ref) <= 2e-2
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=2e-2, atol=5e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_long_rows_empty_molecule_and_mask_holes(cuda, dtype):
    # mask rows longer than 252 bytes (several 16-byte chunks per scanned
    # segment), a molecule without valid atoms, a hole in the key mask and one
    # in the query mask (neither mask of molecule 2 is a prefix)
    B, H, N, D = 3, 2, 270, 32
    case = list(random_simplicial(B, H, N, D, seed=21, counts=[200, 0, 75], holes=[(2, 10)], std=0.05))
    case[5] = case[5].clone()
    case[5][2, 30] = False
    out, lse, out32, ref, ref_lse = run(tuple(case), cuda, dtype)
    assert torch.isfinite(out32).all()
    for b in range(B):
        assert rel(out32[b].cpu().numpy(), ref[b]) <= 2e-2, b
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=2e-2, atol=5e-2)
    qv = case[5]
    assert torch.count_nonzero(out32.cpu().permute(0, 2, 1, 3)[~qv]) == 0
    assert torch.count_nonzero(out.float().cpu().permute(0, 2, 1, 3)[~qv]) == 0


def test_more_units_than_workgroups(cuda):
    # 256 molecules x 4 heads: more (molecule, head) pairs than the persistent
    # grid has workgroups, molecules of 0 .. 12 atoms, some with holes
    B, H, N, D = 256, 4, 12, 16
    gen = torch.Generator().manual_seed(6)
    counts = torch.randint(0, N + 1, (B,), generator=gen).tolist()
    holes = [(b, 1) for b in range(0, B, 7) if counts[b] > 2]
    case = random_simplicial(B, H, N, D, seed=9, counts=counts, holes=holes, std=0.3)
    out, lse, out32, ref, ref_lse = run(case, cuda, torch.bfloat16)
    assert rel(out32.cpu().numpy(), ref) <= 2e-2
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=2e-2, atol=5e-2)
    qv = case[5]
    assert torch.count_nonzero(out32.cpu().permute(0, 2, 1, 3)[~qv]) == 0
    # a second call reuses the workspace counter from where the first ended
    out2 = run(case, cuda, torch.bfloat16)[2]
    assert torch.equal(out2, out32)


def test_graph_replays_match_eager(cuda):
    # A captured call replays with the same kernel arguments; the unit-claim
    # counter in the workspace is put back to 0 by each launch's last claim,
    # so every replay schedules like a fresh call.  Eager calls run between
    # the replays, and every replay is checked against the eager result.
    B, H, N, D = 6, 2, 40, 64
    q, k1, v1, k2, v2, qv, pkv, _ = random_simplicial(B, H, N, D, seed=31, counts=[40, 33, 17, 2, 25, 39],
                                                      std=0.1)
    ops = [t.to(torch.bfloat16).to(cuda) for t in (q, k1, v1, k2, v2)]
    masks = dict(query_valid=qv.to(cuda), pair_key_valid=pkv.to(cuda), pair_valid=None, precision="bf16_tc")
    eager = hip_simplicial_attention_forward(*ops, **masks)[2].clone()
    side = torch.cuda.Stream(cuda)
    side.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(side):
        warm = hip_simplicial_attention_forward(*ops, **masks)[2]  # workspace of this stream, zeroed, outside capture
    torch.cuda.current_stream(cuda).wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(warm, eager)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        captured = hip_simplicial_attention_forward(*ops, **masks)[2]
    for rep in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), rep
        again = hip_simplicial_attention_forward(*ops, **masks)[2]
        torch.cuda.synchronize()
        assert torch.equal(again, eager), rep
