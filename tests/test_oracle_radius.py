"""Pins the CPU radius oracle (oracle/radius.c, oracle/radius.py).

* non-periodic d^2: bitwise equal to the reference adapter's ``pair_dist2``
  (geometry/adapters.py:98-99; golden vectors written from the reference);
* periodic d^2: the reference's minimum-image ``pair_dist2``
  (adapters.py:176-190) within float32 rounding (the reference contracts the
  quadratic form with einsum in its own order; the oracle fixes one order);
* the Gram matrix of a y1 lattice (lattice.py:32-47,94-100) against the
  reference's;
* the minimum-image KAT of the reference (tests/test_geometry.py:30-39);
* 27 images against a brute force over the 5x5x5 image shell, and bitwise
  symmetry d^2(i,j) == d^2(j,i);
* the bit mask and block mask against their definition on the d^2 matrix;
* the float64 masked attention against torch's scaled_dot_product_attention
  with a boolean mask, and the closed form of an all-equal-logit row.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.native import pair_d2, radius_mask, unpack_bits
from oracle.radius import lattice_y1_to_gram, masked_attention_fp64

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_nonperiodic_d2_bitwise_equal_reference_golden():
    z = np.load(GOLDEN / "geometry_nonperiodic.npz")
    d2 = pair_d2(z["coords"])
    pad = z["pad_mask"]
    valid = ~pad[:, :, None] & ~pad[:, None, :]
    np.testing.assert_array_equal(d2[valid], z["pair_dist2"][valid])


def test_periodic_d2_matches_reference_golden():
    z = np.load(GOLDEN / "geometry_periodic.npz")
    d2 = pair_d2(z["frac"], gram=z["gram"], pbc_radius=1)
    ref = z["pair_dist2"].astype(np.float64)
    scale = np.trace(z["gram"], axis1=1, axis2=2)[:, None, None]  # |G| sets the rounding scale
    err = np.abs(d2 - ref) / np.maximum(ref, 1e-3 * scale)
    assert err.max() <= 2e-6, err.max()
    # the diagonal is exactly 0 in both
    for b in range(d2.shape[0]):
        assert (np.diag(d2[b]) == 0).all()


def test_gram_of_y1_lattice_matches_reference():
    z = np.load(GOLDEN / "geometry_periodic.npz")
    g = lattice_y1_to_gram(z["lattice_y1"])
    np.testing.assert_allclose(g, z["gram"], rtol=2e-6, atol=1e-4)


def test_minimum_image_kat():
    # tests/test_geometry.py:30-39 of the reference: identity cell (y1 = 0),
    # x = [0.1, 0, 0], [0.9, 0, 0] -> minimum-image distance 0.2
    frac = np.array([[[0.1, 0.0, 0.0], [0.9, 0.0, 0.0]]], np.float32)
    gram = lattice_y1_to_gram(np.zeros((1, 6), np.float32))
    np.testing.assert_allclose(gram[0], np.eye(3), atol=1e-6)
    d2 = pair_d2(frac, gram=gram)
    np.testing.assert_allclose(np.sqrt(d2[0, 0, 1]), 0.2, atol=1e-6)
    np.testing.assert_allclose(np.sqrt(d2[0, 1, 0]), 0.2, atol=1e-6)
    bits, _ = radius_mask(frac, 0.25, gram=gram)
    assert unpack_bits(bits, 2)[0].all()
    bits, _ = radius_mask(frac, 0.15, gram=gram)
    np.testing.assert_array_equal(unpack_bits(bits, 2)[0], np.eye(2, dtype=bool))


def test_27_images_equal_the_5x5x5_shell_and_are_symmetric():
    z = np.load(GOLDEN / "geometry_periodic.npz")
    d1 = pair_d2(z["frac"], gram=z["gram"], pbc_radius=1)
    d2 = pair_d2(z["frac"], gram=z["gram"], pbc_radius=2)
    # cells with angles in [80, 100] degrees: the minimum image is always
    # among the 27 nearest offsets, and every image value is computed the
    # same way in both searches
    np.testing.assert_array_equal(d1, d2)
    np.testing.assert_array_equal(d1, d1.transpose(0, 2, 1))


def _nearest_image_mask(frac, gram, cutoff, R, clamp):
    """The GPU kernel's one-image shortcut, restated in float32 numpy: offset
    o = -rint(d), clamped to {-R..R} when ``clamp``, evaluated in the oracle's
    operation order."""
    f32 = np.float32
    d = (frac[:, :, None, :] - frac[:, None, :, :]).astype(f32)
    o = -np.rint(d)
    if clamp:
        o = np.clip(o, -R, R)
    e = (d + o.astype(f32)).astype(f32)
    G = gram[:, None, None].astype(f32)
    t = [((G[..., c, 0] * e[..., 0]).astype(f32) + (G[..., c, 1] * e[..., 1]).astype(f32)).astype(f32)
         + (G[..., c, 2] * e[..., 2]).astype(f32) for c in range(3)]
    t = [x.astype(f32) for x in t]
    s = ((e[..., 0] * t[0]).astype(f32) + (e[..., 1] * t[1]).astype(f32)).astype(f32)
    s = (s + (e[..., 2] * t[2]).astype(f32)).astype(f32)
    return s <= f32(cutoff) * f32(cutoff)


@pytest.mark.parametrize("R", [1, 2])
def test_nearest_image_shortcut_needs_the_offset_clamp(R):
    """For cells whose image bounds are all below 1/2 the kernel evaluates one
    image per pair.  The reference searches only offsets {-R..R}
    (adapters.py:141-149) and does not wrap fractional coordinates, so the
    shortcut equals the full search only with the offset clamped to that
    range; unwrapped coordinates tell the two apart."""
    rng = np.random.default_rng(20 + R)
    B, N, cutoff = 2, 200, 6.0
    frac = rng.uniform(-2.5, 3.5, (B, N, 3)).astype(np.float32)
    y1 = np.concatenate([np.log(rng.uniform(15, 30, (B, 3))), np.cos(np.deg2rad(rng.uniform(80, 100, (B, 3))))],
                        axis=1).astype(np.float32)
    gram = lattice_y1_to_gram(y1)
    bits, _ = radius_mask(frac, cutoff, gram=gram, pbc_radius=R)
    full = unpack_bits(bits, N)
    assert 0.003 < full.mean() < 0.2
    np.testing.assert_array_equal(_nearest_image_mask(frac, gram, cutoff, R, clamp=True), full)
    assert (_nearest_image_mask(frac, gram, cutoff, R, clamp=False) != full).sum() > 100


@pytest.mark.parametrize("periodic", [False, True])
def test_bit_mask_and_block_mask_follow_their_definition(periodic):
    rng = np.random.default_rng(3 + periodic)
    B, N, block = 3, 150, 64
    if periodic:
        coords = rng.random((B, N, 3)).astype(np.float32)
        y1 = np.concatenate([np.log(rng.uniform(8, 12, (B, 3))), np.cos(np.deg2rad(rng.uniform(80, 100, (B, 3))))],
                            axis=1).astype(np.float32)
        gram = lattice_y1_to_gram(y1)
        cutoff = 4.0
    else:
        coords = (rng.standard_normal((B, N, 3)) * 3).astype(np.float32)
        gram = None
        cutoff = 3.0
    pad = np.zeros((B, N), bool)
    pad[1, 100:] = True
    pad[2, ::5] = True
    bits, blocks = radius_mask(coords, cutoff, gram=gram, pad_mask=pad, block=block)
    d2 = pair_d2(coords, gram=gram)
    valid = ~pad[:, :, None] & ~pad[:, None, :]
    expect = (d2 <= np.float32(cutoff) * np.float32(cutoff)) & valid
    m = unpack_bits(bits, N)
    np.testing.assert_array_equal(m, expect)
    assert 0.02 < expect[valid].mean() < 0.5  # the case exercises both outcomes
    # padding bits beyond N stay 0
    W = bits.shape[-1]
    full = unpack_bits(bits, W * 32)
    assert not full[..., N:].any()
    NB = (N + block - 1) // block
    for b in range(B):
        for bi in range(NB):
            for bj in range(NB):
                tile = expect[b, bi * block:(bi + 1) * block, bj * block:(bj + 1) * block]
                assert blocks[b, bi, bj] == tile.any()
    # every valid atom is its own neighbour
    for b in range(B):
        assert (np.diag(m[b]) == ~pad[b]).all()


def test_masked_attention_matches_sdpa_and_closed_form():
    rng = np.random.default_rng(7)
    B, H, N, D = 2, 3, 20, 8
    q, k, v = (rng.standard_normal((B, H, N, D)) for _ in range(3))
    mask = rng.random((B, N, N)) < 0.3
    mask |= np.eye(N, dtype=bool)[None]
    mask[1, 15:, :] = False  # rows without any allowed key
    scale = D ** -0.5
    out, lse = masked_attention_fp64(q, k, v, mask, scale)
    has = mask.any(-1)
    tq, tk, tv = (torch.from_numpy(a) for a in (q, k, v))
    tm = torch.from_numpy(mask)[:, None]
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=tm, scale=scale)
    ref = torch.where(torch.from_numpy(has)[:, None, :, None], ref, torch.zeros(()))
    np.testing.assert_allclose(out, ref.numpy(), atol=1e-12)
    s = np.einsum("bhid,bhjd->bhij", q, k) * scale
    with np.errstate(divide="ignore"):
        ref_lse = np.log(np.where(mask[:, None], np.exp(s), 0).sum(-1))
    np.testing.assert_allclose(lse[np.broadcast_to(has[:, None], lse.shape)],
                               ref_lse[np.broadcast_to(has[:, None], lse.shape)], rtol=1e-12)
    assert (out[1, :, 15:] == 0).all() and (lse[1, :, 15:] == 0).all()
    # q = 0: every allowed logit equal -> the mean of the allowed v_j
    out0, _ = masked_attention_fp64(np.zeros_like(q), k, v, mask, scale)
    mean = np.einsum("bij,bhjd->bhid", mask / np.maximum(mask.sum(-1, keepdims=True), 1), v)
    np.testing.assert_allclose(out0, mean, atol=1e-12)
