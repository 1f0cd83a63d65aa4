"""SimplicialGeometryBias (matterformer_amd.geometry_bias) against the fixture written from the reference module
(transformer.py:516-996) by the shared procedure of geometry_bias_fixture.py: seeded construction and first call
draw the same weights (parameter checksums equal), and every output -- u, v, w, the noise gate, the attention
mask, the low-rank angle and message factors, the dense angle residual -- matches the reference's on the same
features (the torch formulation, on the CPU)."""

import numpy as np
import pytest
import torch

import geometry_bias_fixture as fx
from matterformer_amd.geometry import GeometryFeatures
from matterformer_amd.geometry_bias import SimplicialGeometryBias, build_simplicial_attention_mask


def _features(z):
    t = {k: torch.from_numpy(z[k]) for k in ("pair_delta", "pair_dist", "pair_dist2", "pair_dist_norm", "pair_mask",
                                            "global_geom")}
    metric = torch.eye(3).expand(t["pair_delta"].shape[0], -1, -1)
    return GeometryFeatures(pair_delta=t["pair_delta"], pair_dist=t["pair_dist"], pair_dist2=t["pair_dist2"],
                            pair_dist_norm=t["pair_dist_norm"], pair_mask=t["pair_mask"],
                            global_geom=t["global_geom"], kind="nonperiodic", extras={"metric": metric})


@pytest.mark.parametrize("case", list(fx.CASES))
def test_mirror_matches_reference_fixture(case):
    z = np.load(fx.GOLDEN)
    feats = _features(z)
    pad = torch.from_numpy(z["pad_mask"])
    sigma = torch.from_numpy(z["sigma"])
    module, result = fx.build(SimplicialGeometryBias, case, feats, pad, sigma)
    assert list(module.state_dict().keys()) == list(z[f"{case}_param_names"])
    np.testing.assert_array_equal(fx.param_checks(module), z[f"{case}_param_checks"])
    got = fx.outputs(result)
    want = {k[len(case) + 1:]: z[k] for k in z.files if k.startswith(case + "_") and "param" not in k}
    assert sorted(got) == sorted(want)
    for k, v in want.items():
        np.testing.assert_allclose(got[k], v, rtol=1e-6, atol=1e-7, err_msg=k)


def test_zero_initialised_module_gives_zero_terms_and_the_noise_gate():
    z = np.load(fx.GOLDEN)
    feats = _features(z)
    sigma = torch.tensor([0.5, 1.0, 2.0])
    m = SimplicialGeometryBias(4, edge_bias_hidden_dim=16)
    fb, fn, angle, msg, mask = m.build_structured_bias_inputs(feats, coords_len=fx.N, sigma=sigma)
    assert fn is None and angle is None and msg is None
    assert not fb.u.any() and not fb.v.any() and not fb.w.any()
    # softplus(alpha_raw) = 1 and beta = 0 at construction: gate = sigmoid(-log sigma)
    torch.testing.assert_close(fb.gate[:, 0, 0], torch.sigmoid(-torch.log(sigma)))
    with pytest.raises(ValueError, match="sigma must be provided"):
        m.build_structured_bias_inputs(feats, coords_len=fx.N)


def test_attention_mask_builder_conventions():
    pad = torch.tensor([[False, False, True, False]])
    geo = torch.ones(1, 3, 3, dtype=torch.bool)
    geo[0, 0, 1] = False
    m = build_simplicial_attention_mask(coords_len=3, seq_len=4, batch_size=1, device=torch.device("cpu"),
                                        pad_mask=pad, geom_pair_mask=geo)
    assert m.query_valid.tolist() == [[True, True, False, True]]
    assert m.pair_key_valid.tolist() == [[True, True, False, False]]  # the 4th token is no atom
    assert m.pair_valid[0, :3, :3].tolist() == geo[0].tolist() and not m.pair_valid[0, 3].any()
    g = build_simplicial_attention_mask(coords_len=3, seq_len=4, batch_size=1, device=torch.device("cpu"),
                                        pad_mask=pad, include_global_tokens_as_pair_keys=True)
    assert g.pair_valid is None and torch.equal(g.pair_key_valid, g.query_valid)
    with pytest.raises(ValueError, match="smaller than coords_len"):
        build_simplicial_attention_mask(coords_len=5, seq_len=4, batch_size=1, device=torch.device("cpu"))
