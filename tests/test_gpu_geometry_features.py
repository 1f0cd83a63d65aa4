"""GPU parity of mf_geometry_features (one-pass pair features) through the adapters of matterformer_amd.geometry.

Bars: non-periodic d2 and delta bit for bit against the reference's fixture (adapters.py:83-125), dist the
correctly rounded square root of d2; periodic delta (the chosen image) bit for bit against the reference's
fixture (adapters.py:151-212), d2 bit for bit against the C oracle's minimum-image d2 (oracle/radius.c,
pinned to the reference's fixture) and within 2e-6 of the reference's einsum; the same pass's cutoff bits
identical to mf_radius_mask's; every output 0 outside the valid pairs.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from matterformer_amd.geometry import NonPeriodicGeometryAdapter, PeriodicGeometryAdapter
from matterformer_amd.geometry_ops import lattice_to_gram, radius_mask
from matterformer_amd.workloads import radius_workload
from oracle.native import pair_d2 as oracle_pair_d2

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def test_nonperiodic_features_match_reference_fixture(cuda):
    z = np.load(GOLDEN / "geometry_nonperiodic.npz")
    coords, pad = torch.from_numpy(z["coords"]), torch.from_numpy(z["pad_mask"])
    f = NonPeriodicGeometryAdapter()(coords.to(cuda), pad_mask=pad.to(cuda))
    cpu = NonPeriodicGeometryAdapter()(coords, pad_mask=pad)
    assert np.array_equal(f.pair_dist2.cpu().numpy(), z["pair_dist2"])
    assert np.array_equal(f.pair_delta.cpu().numpy(), cpu.pair_delta.numpy())
    d2 = z["pair_dist2"].astype(np.float64)
    assert np.array_equal(f.pair_dist.cpu().numpy(), np.sqrt(d2).astype(np.float32))
    np.testing.assert_allclose(f.pair_dist_norm.cpu().numpy(), cpu.pair_dist_norm.numpy(), rtol=1e-6, atol=0)


def test_periodic_features_match_reference_fixture(cuda):
    z = np.load(GOLDEN / "geometry_periodic.npz")
    frac, lat = torch.from_numpy(z["frac"]), torch.from_numpy(z["lattice_y1"])
    f = PeriodicGeometryAdapter()(frac.to(cuda), lattice=lat.to(cuda))
    assert np.array_equal(f.pair_delta.cpu().numpy(), z["pair_delta"])
    np.testing.assert_allclose(f.pair_dist2.cpu().numpy(), z["pair_dist2"], rtol=2e-6, atol=1e-6)
    gram = lattice_to_gram(lat.to(cuda)).cpu().numpy()
    assert np.array_equal(f.pair_dist2.cpu().numpy(), oracle_pair_d2(z["frac"], gram, 1))


@pytest.mark.parametrize("pbc_radius,rep", [(1, "y1"), (2, "y1"), (1, "ltri")])
def test_periodic_features_with_padding_match_cpu_path(cuda, pbc_radius, rep):
    gen = torch.Generator().manual_seed(31 + pbc_radius)
    B, N = 3, 75
    frac = torch.rand(B, N, 3, generator=gen) * 1.4 - 0.2   # outside [0, 1) too
    if rep == "y1":
        lat = torch.cat([torch.log(8.0 + 10.0 * torch.rand(B, 3, generator=gen)),
                         torch.cos((70.0 + 40.0 * torch.rand(B, 3, generator=gen)) * np.pi / 180.0)], dim=-1)
    else:
        lat = torch.cat([torch.log(6.0 + 6.0 * torch.rand(B, 1, generator=gen)), torch.randn(B, 1, generator=gen),
                         torch.log(6.0 + 6.0 * torch.rand(B, 1, generator=gen)), torch.randn(B, 2, generator=gen),
                         torch.log(6.0 + 6.0 * torch.rand(B, 1, generator=gen))], dim=-1)
    pad = torch.rand(B, N, generator=gen) < 0.15
    ad = PeriodicGeometryAdapter(pbc_radius=pbc_radius, lattice_repr=rep)
    f = ad(frac.to(cuda), pad_mask=pad.to(cuda), lattice=lat.to(cuda), radius_cutoff=5.0)
    cpu = ad(frac, pad_mask=pad, lattice=lat, radius_cutoff=5.0)
    gram = lattice_to_gram(lat.to(cuda), rep)
    d2_oracle = oracle_pair_d2(frac.numpy(), gram.cpu().numpy(), pbc_radius)
    pm = cpu.pair_mask.numpy()
    assert np.array_equal(f.pair_dist2.cpu().numpy(), np.where(pm, d2_oracle, 0.0).astype(np.float32))
    np.testing.assert_allclose(f.pair_dist2.cpu().numpy(), cpu.pair_dist2.numpy(), rtol=5e-6, atol=1e-5)
    # the image choice agrees with the reference formulation except on numerical ties between images
    same = (f.pair_delta.cpu() == cpu.pair_delta).all(dim=-1).numpy()
    assert same.mean() > 0.999
    assert not f.pair_dist2.cpu().numpy()[~pm].any() and not f.pair_delta.cpu().numpy()[~pm].any()
    bits, _ = radius_mask(frac.to(cuda), 5.0, gram=gram, pad_mask=pad.to(cuda), pbc_radius=pbc_radius)
    assert torch.equal(f.extras["radius_mask_bits"], bits)


def test_c4_features_and_mask_in_one_pass(cuda):
    """configs[3] cells: the features pass's cutoff bits equal mf_radius_mask's bit for bit."""
    w = radius_workload()
    frac, lat = w.frac.to(cuda), w.lattice.to(cuda)
    f = PeriodicGeometryAdapter()(frac, lattice=lat, radius_cutoff=w.cutoff)
    bits, _ = radius_mask(frac, w.cutoff, gram=lattice_to_gram(lat))
    assert torch.equal(f.extras["radius_mask_bits"], bits)
    assert torch.isfinite(f.pair_dist_norm).all()


def _lattice_cases(seed: int) -> torch.Tensor:
    """Lattice latents: ordinary cells, every clamp engaged (log lengths past +-5, cosines past +-1,
    ltri off-diagonals past +-10) and cells whose third row is degenerate (sqrt of a negative: NaN in the
    cell, 0 in the metric)."""
    gen = torch.Generator().manual_seed(seed)
    lat = torch.cat([torch.rand(64, 3, generator=gen) * 1.5 + 1.8, torch.rand(64, 3, generator=gen) * 0.6 - 0.3],
                    dim=-1)
    wild = torch.randn(64, 6, generator=gen) * 8.0
    degenerate = torch.tensor([[2.0, 2.0, 2.0, 0.9999, -0.9999, 0.9999], [1.0, 1.5, 2.0, -1.0, 1.0, -1.0]])
    return torch.cat([lat, wild, degenerate])


@pytest.mark.parametrize("rep", ["y1", "ltri"])
def test_lattice_terms_kernel_matches_torch_formulation(cuda, rep):
    """mf_lattice_terms (gram, y1, cell scale in one launch) against the torch formulation of
    lattice.py:12-131 / adapters.py:192 on the CPU, and (y1) the metric against the float64 oracle:
    the kernel evaluates the same fp32 operations in the same order, so only exp / log / sqrt rounding
    may differ (relative 1e-6); metric entries the torch formulation zeroes (non-finite) are zero."""
    from matterformer_amd.geometry_ops import _lattice_terms_torch, lattice_terms
    from oracle.radius import lattice_y1_to_gram

    lat = _lattice_cases(17 if rep == "y1" else 18)
    g, y1, sc = (t.cpu() for t in lattice_terms(lat.to(cuda), rep))
    rg, ry1, rsc = _lattice_terms_torch(lat, rep)
    np.testing.assert_allclose(g.numpy(), rg.numpy(), rtol=1e-6, atol=1e-6)
    # (ltri: y1[:3] = log |row| is near 0 for rows of length ~1, where one ulp of the length is ~1.2e-7 absolute)
    np.testing.assert_allclose(y1.numpy(), ry1.numpy(), rtol=1e-6, atol=3e-7)
    np.testing.assert_allclose(sc.numpy(), rsc.numpy(), rtol=1e-6, atol=0)
    assert torch.equal(g == 0, rg == 0)
    assert torch.isfinite(g).all() and torch.isfinite(y1).all() and torch.isfinite(sc).all()
    if rep == "y1":
        ordinary = lat[:64].numpy()
        np.testing.assert_allclose(g[:64].numpy(), lattice_y1_to_gram(ordinary), rtol=2e-6, atol=1e-5)


def test_periodic_adapter_lattice_extras_match_cpu(cuda):
    """The adapter's metric and cell scale (now from mf_lattice_terms) against its CPU formulation."""
    z = np.load(GOLDEN / "geometry_periodic.npz")
    frac, lat = torch.from_numpy(z["frac"]), torch.from_numpy(z["lattice_y1"])
    f = PeriodicGeometryAdapter()(frac.to(cuda), lattice=lat.to(cuda))
    cpu = PeriodicGeometryAdapter()(frac, lattice=lat)
    for key in ("metric", "cell_scale"):
        np.testing.assert_allclose(f.extras[key].cpu().numpy(), cpu.extras[key].numpy(), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(f.global_geom.cpu().numpy(), cpu.global_geom.numpy(), rtol=1e-6, atol=0)
