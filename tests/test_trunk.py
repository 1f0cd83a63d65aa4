"""The configs[4] trunk on the CPU against the fixture written from 12 reference AdaLNBlocks.

tests/golden/trunk_alternating_b4.npz holds the output of the reference's blocks
(src/matterformer/models/transformer.py:154-316; simplicial on even layers, MHA with a kNN 0/-inf
attn_head_bias on odd layers, :256-268) over 4 GEOM-shaped molecules, fp32, plus per-parameter checksums.
Here: the seeded construction reproduces the reference's parameters (names and checksums), the kNN
mask reproduces the fixture's (from the reference's own pair distances), and the torch path of the
trunk reproduces the reference's output.
"""

import numpy as np
import torch

from matterformer_amd.trunk import knn_allowed_torch, knn_lists_torch
from trunk_fixture import build_trunk, inputs, load, valid_rel_err


def test_seeded_construction_reproduces_reference_parameters():
    z = load()
    trunk = build_trunk(z)
    for parity, blocks, key in ((0, trunk.blocks[0::2], "even"), (1, trunk.blocks[1::2], "odd")):
        assert list(blocks[0].state_dict().keys()) == [str(n) for n in z[f"param_names_{key}"]]
        for layer, blk in enumerate(blocks):
            got = np.array([[float(t.double().sum()), float(t.double().square().sum())]
                            for t in blk.state_dict().values()])
            np.testing.assert_allclose(got, z[f"param_checks_{key}"][layer], rtol=1e-12, atol=1e-12,
                                       err_msg=f"{key} block {layer}")


def test_knn_mask_matches_reference_distances():
    z = load()
    _, _, coords, pad = inputs(z)
    idx = knn_lists_torch(coords, int(z["shape"][4]), pad)
    allowed = knn_allowed_torch(idx, pad).numpy()
    valid = ~z["pad_mask"]
    assert np.array_equal(allowed[valid], z["allowed"][valid])
    assert not allowed[~valid].any()


def test_torch_path_matches_reference_blocks():
    z = load()
    trunk = build_trunk(z, simplicial_impl="torch", local_impl="torch", simplicial_precision="ieee_fp32")
    x, cond, coords, pad = inputs(z)
    with torch.no_grad():
        out = trunk(x, cond, coords, pad)
    assert valid_rel_err(out.numpy(), z) <= 1e-5


def test_token_packing_round_trips():
    from matterformer_amd.trunk import TokenPacking

    gen = torch.Generator().manual_seed(3)
    B, N, C, H, D = 3, 7, 10, 2, 8
    pad = torch.rand(B, N, generator=gen) < 0.4
    pad[1] = True  # a molecule with no valid atom
    pad[2, 0] = False
    p = TokenPacking(pad)
    valid = [(b, n) for b in range(B) for n in range(N) if not pad[b, n]]
    W = int((~pad).sum(1).max())
    assert p.tokens == len(valid) and p.width == W
    pos = {}
    for b, n in valid:
        pos[(b, n)] = sum(1 for m in range(n) if not pad[b, m])
    assert [(int(m), int(r) % N) for m, r in zip(p.mol, p.rows)] == valid
    assert [int(q) for q in p.pos] == [pos[v] for v in valid]
    assert torch.equal(p.compact_pad_mask, torch.arange(W)[None, :] >= (~pad).sum(1)[:, None])
    x = torch.randn(B, N, C, generator=gen)
    xp = p.pack(x)
    assert torch.equal(xp, torch.stack([x[b, n] for b, n in valid]))
    back = p.unpack(xp)
    assert torch.equal(back[~pad], x[~pad]) and not back[pad].any()
    xc = p.compact(x)
    assert xc.shape == (B, W, C)
    for b, n in valid:
        assert torch.equal(xc[b, pos[(b, n)]], x[b, n])
    assert not xc[p.compact_pad_mask].any()
    per_mol = torch.randn(B, C, generator=gen)
    assert torch.equal(p.per_token(per_mol), torch.stack([per_mol[b] for b, _ in valid]))
    proj = torch.randn(p.tokens, 3 * H * D, generator=gen)
    heads = p.to_heads(proj, 3, H, D, torch.float64, first_part_scale=0.5)
    assert heads.shape == (3, B, H, W, D) and heads.dtype == torch.float64
    for t, (b, n) in enumerate(valid):
        want = proj[t].view(3, H, D).double().clone()
        want[0] = (proj[t].view(3, H, D)[0] * 0.5).double()
        assert torch.equal(heads[:, b, :, pos[(b, n)], :], want)
    assert not heads.permute(1, 3, 0, 2, 4)[p.compact_pad_mask].any()
    assert torch.equal(p.from_heads(heads[1]), proj[:, H * D:2 * H * D].double())


def test_adaln_rows_torch_expressions():
    """adaln_rows (CPU path) is transformer.py:296-316's torch expressions on the packed rows."""
    from matterformer_amd.token_packing import adaln_rows
    from matterformer_amd.trunk import TokenPacking

    gen = torch.Generator().manual_seed(5)
    B, N, C = 3, 6, 16
    pad = torch.rand(B, N, generator=gen) < 0.3
    p = TokenPacking(pad)
    for dtype in (torch.float32, torch.bfloat16):
        x = torch.randn(B, N, C, generator=gen).to(dtype)
        y = torch.randn(B, N, C, generator=gen).to(dtype)
        mods = (torch.randn(B, 6 * C, generator=gen) * 0.3).to(dtype)
        sh, sc, g = mods[:, :C], mods[:, C:2 * C], mods[:, 2 * C:3 * C]
        xr = x + g[:, None, :] * y
        hr = torch.nn.functional.layer_norm(xr, (C,), eps=1e-6) * (1.0 + sc[:, None, :]) + sh[:, None, :]
        xo, h = adaln_rows(p, p.pack(x), p.pack(y), gate=g, shift=sh, scale=sc, eps=1e-6)
        assert torch.equal(xo, xr[~pad]) and torch.equal(h, hr[~pad])
        only_h = adaln_rows(p, p.pack(x), shift=sh, scale=sc, eps=1e-6)
        hx = torch.nn.functional.layer_norm(x, (C,), eps=1e-6) * (1.0 + sc[:, None, :]) + sh[:, None, :]
        assert torch.equal(only_h, hx[~pad])
        assert torch.equal(adaln_rows(p, p.pack(x), p.pack(y), gate=g), xr[~pad])


def test_torch_path_zeroes_padded_rows():
    """transformer.py:1298-1316: the trunk output is zero on padded atoms."""
    z = load()
    trunk = build_trunk(z, local_impl="torch", simplicial_impl="torch")
    x, cond, coords, pad = inputs(z)
    with torch.no_grad():
        out = trunk(x[:2], cond[:2], coords[:2], pad[:2])
    assert not out[pad[:2]].any()
    assert out[~pad[:2]].abs().sum() > 0


def test_compact_dims_and_terms_follow_the_packing():
    """TokenPacking.compact_dims moves atom axes N -> W (valid atoms first, zero / False past the count), on
    every named axis; SimplicialTerms.compact applies it to the mask and each term."""
    from matterformer_amd.simplicial_types import (SimplicialAttentionMask, SimplicialFactorizedBias,
                                                   SimplicialLowRankAngleResidual)
    from matterformer_amd.trunk import SimplicialTerms, TokenPacking

    gen = torch.Generator().manual_seed(9)
    B, H, N, R = 3, 2, 6, 3
    pad = torch.rand(B, N, generator=gen) < 0.4
    pad[0] = False
    p = TokenPacking(pad)
    W = p.width
    idx = [[n for n in range(N) if not pad[b, n]] for b in range(B)]
    u = torch.randn(B, H, N, N, generator=gen)
    got = p.compact_dims(u, 2, 3)
    assert got.shape == (B, H, W, W)
    for b in range(B):
        c = len(idx[b])
        want = torch.zeros(H, W, W)
        want[:, :c, :c] = u[b][:, idx[b]][:, :, idx[b]]
        assert torch.equal(got[b], want)
    pv = torch.rand(B, N, N, generator=gen) < 0.7
    gpv = p.compact_dims(pv, 1, 2)
    for b in range(B):
        c = len(idx[b])
        assert torch.equal(gpv[b, :c, :c], pv[b][idx[b]][:, idx[b]])
        assert not gpv[b, c:].any() and not gpv[b, :, c:].any()
    left = torch.randn(B, H, N, N, R, generator=gen)
    gate = torch.rand(B, H, 1, generator=gen).expand(B, H, N)
    mask = SimplicialAttentionMask(query_valid=~pad, pair_key_valid=~pad, pair_valid=pv)
    terms = SimplicialTerms(mask, SimplicialFactorizedBias(u=u, v=u * 2, w=-u, gate=gate),
                            SimplicialLowRankAngleResidual(left=left, right=left * 3, gate=gate))
    ct = terms.compact(p)
    assert torch.equal(ct.attention_mask.query_valid, ~p.compact_pad_mask)
    assert torch.equal(ct.attention_mask.pair_valid, gpv)
    assert torch.equal(ct.factorized_bias.w, -got)
    assert torch.equal(ct.factorized_bias.gate, gate[:, :, :W] * (~p.compact_pad_mask)[:, None, :])
    assert ct.angle_residual.left.shape == (B, H, W, W, R)
    assert torch.equal(ct.angle_residual.right, p.compact_dims(left * 3, 2, 3))


def test_geometry_trunk_valid_rows_ignore_padded_atoms():
    """With a geometry adapter and SimplicialGeometryBias (angle_low_rank + low-rank message), the torch
    trunk's valid rows do not depend on the padded atoms' features or coordinates, padded rows are zero, and
    the bias terms do reach the output."""
    from trunk_fixture import geometry_inputs, geometry_trunk

    trunk = geometry_trunk()
    x, cond, coords, pad, sigma = geometry_inputs()
    with torch.no_grad():
        out = trunk(x, cond, coords, pad, sigma=sigma)
        x2, c2 = x.clone(), coords.clone()
        x2[pad] = 7.0
        c2[pad] = -3.0
        out2 = trunk(x2, cond, c2, pad, sigma=sigma)
        for prm in trunk.simplicial_geometry_bias.spoke_bias_u_mlp.parameters():
            prm.data.mul_(2.0)
        out3 = trunk(x, cond, coords, pad, sigma=sigma)
    assert all(b.attn._last_impl_used == "torch" for b in trunk.blocks if b.attn_type == "simplicial")
    assert not out[pad].any() and not out2[pad].any()
    torch.testing.assert_close(out2[~pad], out[~pad], rtol=1e-5, atol=1e-5)
    assert float((out3 - out)[~pad].abs().max()) > 1e-3
