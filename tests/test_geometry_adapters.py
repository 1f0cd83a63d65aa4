"""The product's geometry adapters (matterformer_amd.geometry) on the CPU against the reference's fixtures.

tests/golden/geometry_*.npz were written by the reference's NonPeriodicGeometryAdapter and
PeriodicGeometryAdapter (src/matterformer/geometry/adapters.py:83-125,151-212).  On CPU tensors the adapters
run the reference's own torch formulation, so d2 and the chosen image's delta are reproduced exactly, the
periodic d2 (an einsum) to rounding.
"""

from pathlib import Path

import numpy as np
import torch

from matterformer_amd.geometry import NonPeriodicGeometryAdapter, PeriodicGeometryAdapter

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_nonperiodic_adapter_matches_reference_fixture():
    z = np.load(GOLDEN / "geometry_nonperiodic.npz")
    f = NonPeriodicGeometryAdapter()(torch.from_numpy(z["coords"]), pad_mask=torch.from_numpy(z["pad_mask"]))
    assert np.array_equal(f.pair_dist2.numpy(), z["pair_dist2"])
    assert np.array_equal(f.pair_dist.numpy(), z["pair_dist"])
    assert f.pair_delta.shape == (3, 37, 37, 3) and f.kind == "nonperiodic"
    pad = z["pad_mask"]
    assert not f.pair_dist2.numpy()[1][pad[1]].any()


def test_periodic_adapter_matches_reference_fixture():
    z = np.load(GOLDEN / "geometry_periodic.npz")
    f = PeriodicGeometryAdapter(pbc_radius=1, lattice_repr="y1")(
        torch.from_numpy(z["frac"]), lattice=torch.from_numpy(z["lattice_y1"]))
    np.testing.assert_allclose(f.pair_dist2.numpy(), z["pair_dist2"], rtol=2e-6, atol=1e-6)
    assert np.array_equal(f.pair_delta.numpy(), z["pair_delta"])
    np.testing.assert_allclose(f.extras["metric"].numpy(), z["gram"], rtol=2e-6, atol=1e-6)
    assert f.global_geom.shape == (3, 6) and f.kind == "periodic"
