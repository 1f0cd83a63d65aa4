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
