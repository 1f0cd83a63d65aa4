"""mf_pair_mlp_bias (the factorized geometry-bias MLPs in one pass) against SimplicialGeometryBias's torch
formulation: the reference-fixture module and a configs[1]-sized batch.  Bar: fp32 MFMA against the fp32 torch
GEMMs, max |difference| <= 1e-5 relative to the largest |term| per head (measured ~1e-6); the diagonal and the
invalid pairs exactly zero.  Its weight backward (mf_pair_mlp_bias_bwd) against float64 autograd of the torch
formulation, normwise 2e-5 per gradient, and bitwise repeatable."""

import numpy as np
import pytest
import torch

import geometry_bias_fixture as fx
from matterformer_amd import pair_mlp
from matterformer_amd.geometry import GeometryFeatures, NonPeriodicGeometryAdapter
from matterformer_amd.geometry_bias import SimplicialGeometryBias
from test_geometry_bias import _features

pytestmark = pytest.mark.gpu


def _to(feats, dev):
    return GeometryFeatures(pair_delta=feats.pair_delta.to(dev), pair_dist=feats.pair_dist.to(dev),
                            pair_dist2=feats.pair_dist2.to(dev), pair_dist_norm=feats.pair_dist_norm.to(dev),
                            pair_mask=feats.pair_mask.to(dev), global_geom=feats.global_geom.to(dev), kind=feats.kind,
                            extras={k: v.to(dev) for k, v in feats.extras.items()})


def _check(got, want, mask):
    for g, w in zip(got, want):
        g, w = g.cpu().double(), w.cpu().double()
        scale = w.abs().amax(dim=(-2, -1), keepdim=True).clamp_min(1e-30)
        err = ((g - w).abs() / scale).max().item()
        assert err <= 1e-5, err
        n = g.shape[-1]
        assert not g[..., torch.arange(n), torch.arange(n)].any()
        assert not g.permute(0, 2, 3, 1)[~mask.cpu()].any()


def test_fixture_module_on_gpu_matches_torch(cuda):
    z = np.load(fx.GOLDEN)
    feats = _features(z)
    module, _ = fx.build(SimplicialGeometryBias, "lowrank", feats, torch.from_numpy(z["pad_mask"]),
                         torch.from_numpy(z["sigma"]))
    want = module._compute_factorized_terms(feats)  # CPU: torch formulation
    module = module.to(cuda)
    gfe = _to(feats, cuda)
    with torch.no_grad():
        assert pair_mlp.serves(module, gfe)
        got = module._compute_factorized_terms(gfe)
    torch.cuda.synchronize()
    _check(got, want, feats.pair_mask)
    np.testing.assert_allclose(got[0].cpu().numpy(), z["lowrank_u"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("B,N,hidden,H,R", [(64, 181, 128, 8, 16), (5, 37, 64, 4, 29), (3, 20, 16, 16, 1)])
def test_configs_sized_batch_matches_torch(cuda, B, N, hidden, H, R):
    print(f"pair mlp B={B} N={N} hidden={hidden} H={H} R={R}", flush=True)
    gen = torch.Generator().manual_seed(B + N)
    counts = torch.randint(max(2, N // 4), N + 1, (B,), generator=gen)
    pad = torch.arange(N)[None, :] >= counts[:, None]
    coords = torch.randn(B, N, 3, generator=gen) * 1.4
    torch.manual_seed(7)
    module = SimplicialGeometryBias(H, edge_bias_hidden_dim=hidden, edge_bias_n_rbf=R)
    feats = NonPeriodicGeometryAdapter()(coords, pad_mask=pad)
    module._compute_factorized_terms(feats)  # materialise the LazyLinear layers
    with torch.no_grad():
        for mlp in (module.spoke_bias_u_mlp, module.spoke_bias_v_mlp, module.pair_bias_w_mlp):
            mlp[2].weight.copy_(torch.randn(mlp[2].weight.shape, generator=gen) * 0.2)
            mlp[2].bias.copy_(torch.randn(mlp[2].bias.shape, generator=gen) * 0.2)
    sub = slice(0, min(B, 6))  # the torch reference on the CPU for a slice of the batch
    want = [t[sub] for t in module._compute_factorized_terms(
        GeometryFeatures(**{k: (getattr(feats, k)[sub] if k not in ("kind", "extras") else getattr(feats, k))
                            for k in ("pair_delta", "pair_dist", "pair_dist2", "pair_dist_norm", "pair_mask",
                                      "global_geom", "kind", "extras")}))]
    module = module.to(cuda)
    gfe = NonPeriodicGeometryAdapter()(coords.to(cuda), pad_mask=pad.to(cuda))
    with torch.no_grad():
        got = module._compute_factorized_terms(gfe)
    torch.cuda.synchronize()
    _check([t[sub] for t in got], want, feats.pair_mask[sub])
    assert all(torch.isfinite(t).all() for t in got)


def _trained_module(B, N, hidden, H, R, seed):
    """A SimplicialGeometryBias with materialised, non-zero layers and its non-periodic features (CPU)."""
    gen = torch.Generator().manual_seed(seed)
    counts = torch.randint(max(2, N // 3), N + 1, (B,), generator=gen)
    pad = torch.arange(N)[None, :] >= counts[:, None]
    coords = torch.randn(B, N, 3, generator=gen) * 1.4
    torch.manual_seed(seed)
    module = SimplicialGeometryBias(H, edge_bias_hidden_dim=hidden, edge_bias_n_rbf=R)
    feats = NonPeriodicGeometryAdapter()(coords, pad_mask=pad)
    with torch.no_grad():
        module._compute_factorized_terms(feats)  # materialise the LazyLinear layers
        for mlp in (module.spoke_bias_u_mlp, module.spoke_bias_v_mlp, module.pair_bias_w_mlp):
            mlp[2].weight.copy_(torch.randn(mlp[2].weight.shape, generator=gen) * 0.2)
            mlp[2].bias.copy_(torch.randn(mlp[2].bias.shape, generator=gen) * 0.2)
    ups = [torch.randn(B, H, N, N, generator=gen) for _ in range(3)]  # non-zero at invalid pairs too
    return module, feats, coords, pad, ups


def _weight_grads(module, feats, ups):
    module.zero_grad(set_to_none=True)
    u, v, w = module._compute_factorized_terms(feats)
    ((u * ups[0]).sum() + (v * ups[1]).sum() + (w * ups[2]).sum()).backward()
    return [p.grad.detach().clone() for m in (module.spoke_bias_u_mlp, module.spoke_bias_v_mlp,
                                              module.pair_bias_w_mlp) for p in (m[0].weight, m[0].bias,
                                                                               m[2].weight, m[2].bias)]


@pytest.mark.parametrize("B,N,hidden,H,R", [(6, 48, 128, 8, 16), (3, 37, 64, 4, 28), (3, 20, 16, 16, 1)])
def test_weight_gradients_match_float64_autograd(cuda, B, N, hidden, H, R):
    """mf_pair_mlp_bias_bwd (through the autograd Function) against float64 autograd of the torch
    formulation on the CPU: the 12 weight gradients of the u, v, w MLPs, normwise relative error <= 2e-5
    per tensor (fp32 MFMA sums over the valid pairs; upstream gradients non-zero at invalid pairs and on the
    diagonal, which must contribute nothing)."""
    import copy

    print(f"pair mlp bwd B={B} N={N} hidden={hidden} H={H} R={R}", flush=True)
    module, feats, coords, pad, ups = _trained_module(B, N, hidden, H, R, seed=B * 7 + N)
    ref_module = copy.deepcopy(module).double()
    feats64 = GeometryFeatures(pair_delta=feats.pair_delta.double(), pair_dist=feats.pair_dist.double(),
                               pair_dist2=feats.pair_dist2.double(), pair_dist_norm=feats.pair_dist_norm.double(),
                               pair_mask=feats.pair_mask, global_geom=feats.global_geom.double(), kind=feats.kind,
                               extras=feats.extras)
    want = _weight_grads(ref_module, feats64, [t.double() for t in ups])
    module = module.to(cuda)
    gfe = NonPeriodicGeometryAdapter()(coords.to(cuda), pad_mask=pad.to(cuda))
    assert pair_mlp.serves(module, gfe)  # grad enabled: the kernel's autograd Function
    got = _weight_grads(module, gfe, [t.to(cuda) for t in ups])
    torch.cuda.synchronize()
    for k, (g, r) in enumerate(zip(got, want)):
        g, r = g.cpu().double(), r.double()
        rel = float((g - r).norm() / r.norm().clamp_min(1e-30))
        assert rel <= 2e-5, (k, rel)


def test_weight_gradients_are_bitwise_deterministic(cuda):
    module, feats, coords, pad, ups = _trained_module(4, 40, 128, 8, 16, seed=5)
    module = module.to(cuda)
    gfe = NonPeriodicGeometryAdapter()(coords.to(cuda), pad_mask=pad.to(cuda))
    ups = [t.to(cuda) for t in ups]
    first = _weight_grads(module, gfe, ups)
    second = _weight_grads(module, gfe, ups)
    assert all(torch.equal(a, b) for a, b in zip(first, second))


def test_grad_calls_outside_the_backward_take_the_torch_path(cuda):
    """Features that take gradients, or 29 rbf features, under autograd: the torch formulation."""
    module, feats, coords, pad, ups = _trained_module(2, 20, 16, 4, 16, seed=9)
    module = module.to(cuda)
    gfe = NonPeriodicGeometryAdapter()(coords.to(cuda), pad_mask=pad.to(cuda))
    assert pair_mlp.serves(module, gfe)
    d = gfe.pair_dist_norm.clone().requires_grad_(True)
    g2 = GeometryFeatures(pair_delta=gfe.pair_delta, pair_dist=gfe.pair_dist, pair_dist2=gfe.pair_dist2,
                          pair_dist_norm=d, pair_mask=gfe.pair_mask, global_geom=gfe.global_geom, kind=gfe.kind,
                          extras=gfe.extras)
    assert not pair_mlp.serves(module, g2)
    with torch.no_grad():
        assert pair_mlp.serves(module, g2)
    m29, f29, c29, p29, _ = _trained_module(2, 20, 16, 4, 29, seed=10)
    m29 = m29.to(cuda)
    g29 = NonPeriodicGeometryAdapter()(c29.to(cuda), pad_mask=p29.to(cuda))
    assert not pair_mlp.serves(m29, g29)
    with torch.no_grad():
        assert pair_mlp.serves(m29, g29)


def test_bias_feeds_hip_attention(cuda):
    """build_structured_bias_inputs on the GPU (kernel u, v, w) into SimplicialAttention's HIP path, against the
    same module on the CPU (torch u, v, w, torch attention)."""
    from matterformer_amd.simplicial_attention import SimplicialAttention

    z = np.load(fx.GOLDEN)
    feats = _features(z)
    pad, sigma = torch.from_numpy(z["pad_mask"]), torch.from_numpy(z["sigma"])
    module, _ = fx.build(SimplicialGeometryBias, "lowrank", feats, pad, sigma)
    module.mode = "factorized"  # only u, v, w for this comparison
    module.message_mode = "none"
    torch.manual_seed(3)
    attn = SimplicialAttention(32, fx.H, precision="ieee_fp32")
    x = torch.randn(fx.B, fx.N, 32)
    with torch.no_grad():
        fb, _, _, _, mask = module.build_structured_bias_inputs(feats, coords_len=fx.N, pad_mask=pad, sigma=sigma)
        want = attn(x, attention_mask=mask, factorized_bias=fb)
        module, attn = module.to(cuda), attn.to(cuda)
        fbg, _, _, _, maskg = module.build_structured_bias_inputs(_to(feats, cuda), coords_len=fx.N,
                                                                  pad_mask=pad.to(cuda), sigma=sigma.to(cuda))
        got = attn(x.to(cuda), attention_mask=maskg, factorized_bias=fbg)
    torch.cuda.synchronize()
    assert attn._last_impl_used == "triton"
    valid = ~pad
    rel = float((got.cpu()[valid] - want[valid]).norm() / want[valid].norm())
    assert rel <= 1e-4, rel


@pytest.mark.parametrize("n_freqs,R", [(8, 16), (2, 5)])
def test_periodic_features_match_torch(cuda, n_freqs, R):
    """use_periodic_features on periodic features (the MOF configuration): the spoke MLPs also read the
    sines / cosines of (2 pi delta_c) freq_k and the cell's 6 global features, the pair MLP the global
    features (transformer.py:641-652).  The same features on both sides (the CPU adapter's, copied to the
    GPU); bar as above (sin / cos in fp32 on both sides)."""
    from matterformer_amd.geometry import PeriodicGeometryAdapter

    gen = torch.Generator().manual_seed(31 + n_freqs)
    B, N, H = 2, 24, 4
    frac = torch.rand(B, N, 3, generator=gen)
    lattice = torch.cat([torch.rand(B, 3, generator=gen) * 0.6 + 2.0, torch.rand(B, 3, generator=gen) * 0.4 - 0.2],
                        dim=-1)
    pad = torch.zeros(B, N, dtype=torch.bool)
    pad[1, 19:] = True
    feats = PeriodicGeometryAdapter()(frac, pad_mask=pad, lattice=lattice)
    torch.manual_seed(4)
    module = SimplicialGeometryBias(H, mode="factorized", edge_bias_hidden_dim=64, edge_bias_n_rbf=R,
                                    edge_bias_n_freqs=n_freqs, use_periodic_features=True)
    with torch.no_grad():
        module._compute_factorized_terms(feats)  # materialise the LazyLinear layers (periodic widths)
        for mlp in (module.spoke_bias_u_mlp, module.spoke_bias_v_mlp, module.pair_bias_w_mlp):
            mlp[2].weight.copy_(torch.randn(mlp[2].weight.shape, generator=gen) * 0.2)
            mlp[2].bias.copy_(torch.randn(mlp[2].bias.shape, generator=gen) * 0.2)
        want = module._compute_factorized_terms(feats)
        module = module.to(cuda)
        gfe = _to(feats, cuda)
        assert pair_mlp.serves(module, gfe)
        got = module._compute_factorized_terms(gfe)
    torch.cuda.synchronize()
    _check(got, want, feats.pair_mask)
    assert not pair_mlp.serves(module, gfe)  # under autograd: the torch formulation (no periodic backward)
