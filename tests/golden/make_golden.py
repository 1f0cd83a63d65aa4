"""Write golden input/output vectors from the stases/Matterformer reference.

Run in the survey container only (the reference is not present on GPU boxes):

    python tests/golden/make_golden.py [/root/reference]

It imports the reference's pure-Python torch path and geometry adapters and
stores small seeded cases as ``.npz`` fixtures next to this script.  The
fixtures pin what the mathematical checks in ``tests/`` leave open: the exact
rounding of the reference's bf16 torch path
(``src/matterformer/models/simplicial_attention.py:161-180,317-329``), its
masking conventions, and the distance / minimum-image conventions of
``src/matterformer/geometry/adapters.py:83-125,151-212``.

bf16 tensors are stored as float32 arrays holding exactly the bf16 values
(the bf16 -> fp32 conversion is exact).
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def _np(t: torch.Tensor) -> np.ndarray:
    t = t.detach()
    if t.dtype in (torch.bfloat16, torch.float16):
        t = t.float()
    return t.cpu().numpy()


def _simplicial_case(ref, name: str, *, seed: int, B: int, H: int, N: int, D: int, dtype: torch.dtype,
                     fp32_core: bool, counts=None, holes=None, pair_drop=0.0, bias=False, angle_rank=0,
                     message_rank=0, chunk_size=128) -> dict:
    gen = torch.Generator().manual_seed(seed)
    scale = 1.0 / math.sqrt(D)
    shape = (B, H, N, D)
    tensors = [(torch.randn(shape, generator=gen) * scale).to(dtype) for _ in range(5)]
    q, k1, v1, k2, v2 = tensors
    key_valid = torch.ones(B, N, dtype=torch.bool)
    if counts is not None:
        for b, n in enumerate(counts):
            key_valid[b, n:] = False
    query_valid = key_valid.clone()
    if holes is not None:  # tokens that are valid queries but not pair keys (CLS-style)
        for b, i in holes:
            key_valid[b, i] = False
    pair_valid = None
    if pair_drop > 0:
        pair_valid = torch.rand(B, N, N, generator=gen) >= pair_drop
    mask = ref.SimplicialAttentionMask(query_valid=query_valid, pair_key_valid=key_valid, pair_valid=pair_valid)
    fb = ar = mr = basis = None
    extra = {}
    if bias:
        fb = ref.SimplicialFactorizedBias(
            u=torch.randn(B, H, N, N, generator=gen).to(dtype),
            v=torch.randn(B, H, N, N, generator=gen).to(dtype),
            w=torch.randn(B, H, N, N, generator=gen).to(dtype),
            gate=torch.randn(B, H, N, generator=gen).to(dtype),
        )
        extra.update(u=_np(fb.u), v_bias=_np(fb.v), w=_np(fb.w), gate=_np(fb.gate))
    if angle_rank:
        ar = ref.SimplicialLowRankAngleResidual(
            left=torch.randn(B, H, N, N, angle_rank, generator=gen).to(dtype),
            right=torch.randn(B, H, N, N, angle_rank, generator=gen).to(dtype),
            gate=torch.randn(B, H, N, generator=gen).to(dtype),
        )
        extra.update(angle_left=_np(ar.left), angle_right=_np(ar.right), angle_gate=_np(ar.gate))
    if message_rank:
        mr = ref.SimplicialLowRankMessageResidual(
            left=torch.randn(B, H, N, N, message_rank, generator=gen).to(dtype),
            right=torch.randn(B, H, N, N, message_rank, generator=gen).to(dtype),
        )
        basis = torch.randn(H, message_rank, D, generator=gen).to(dtype)
        extra.update(message_left=_np(mr.left), message_right=_np(mr.right), message_basis=_np(basis))
    out = ref.simplicial_attention_torch_from_projected(
        q, k1, v1, k2, v2, attention_mask=mask, factorized_bias=fb, angle_residual=ar,
        message_residual=mr, message_basis=basis, chunk_size=chunk_size, fp32_core=fp32_core,
    )
    case = dict(
        q=_np(q), k1=_np(k1), v1=_np(v1), k2=_np(k2), v2=_np(v2),
        query_valid=query_valid.numpy(), pair_key_valid=key_valid.numpy(),
        out=_np(out),
        dtype=np.array(str(dtype).replace("torch.", "")),
        out_dtype=np.array(str(out.dtype).replace("torch.", "")),
        fp32_core=np.array(fp32_core), chunk_size=np.array(chunk_size),
        **extra,
    )
    if pair_valid is not None:
        case["pair_valid"] = pair_valid.numpy()
    np.savez_compressed(HERE / f"simplicial_{name}.npz", **case)
    return case


# Trunk case (configs[4] at a reduced batch): ada_ln's zero-initialised last layer is replaced by
# N(0, TRUNK_ADA_STD^2) draws from torch.Generator().manual_seed(TRUNK_SEED + 100), block by block,
# weight then bias, so that the gates are non-zero (at zero they hide the attention entirely).
TRUNK_SEED = 4
TRUNK_ADA_STD = 0.05
TRUNK_SHAPE = dict(batch=4, d_model=512, heads=8, layers=12, knn_k=32)


def trunk_case(transformer, geometry) -> None:
    """12 reference AdaLNBlocks, simplicial on even and MHA with a kNN 0/-inf attn_head_bias on odd layers
    (transformer.py:154-316, :256-268), fp32 on the CPU.  The kNN uses the reference's own pair distances
    (NonPeriodicGeometryAdapter, adapters.py:98-100): the k nearest valid j != i by (d2, j), plus i itself."""
    B, d, H, L, k = (TRUNK_SHAPE[n] for n in ("batch", "d_model", "heads", "layers", "knn_k"))
    gen = torch.Generator().manual_seed(TRUNK_SEED)
    z = torch.randn(B, generator=gen)
    counts = torch.clamp(torch.round(44.0 + 12.0 * z), 10, 181).to(torch.int64)
    N = int(counts.max())
    pad = torch.arange(N)[None, :] >= counts[:, None]
    x = torch.randn(B, N, d, generator=gen)
    cond = torch.randn(B, d, generator=gen)
    coords = torch.randn(B, N, 3, generator=gen) * math.sqrt(2.0)

    torch.manual_seed(TRUNK_SEED)
    blocks = [transformer.AdaLNBlock(d, H, attn_type="simplicial" if layer % 2 == 0 else "mha",
                                     simplicial_impl="torch", simplicial_precision="ieee_fp32")
              for layer in range(L)]
    ada = torch.Generator().manual_seed(TRUNK_SEED + 100)
    for blk in blocks:
        lin = blk.ada_ln[-1]
        lin.weight.data.copy_(torch.randn(lin.weight.shape, generator=ada) * TRUNK_ADA_STD)
        lin.bias.data.copy_(torch.randn(lin.bias.shape, generator=ada) * TRUNK_ADA_STD)

    d2 = geometry.NonPeriodicGeometryAdapter()(coords, pad_mask=pad).pair_dist2.clone()
    eye = torch.eye(N, dtype=torch.bool)[None]
    d2 = d2.masked_fill(eye | pad[:, None, :] | pad[:, :, None], float("inf"))
    order = torch.sort(d2, dim=-1, stable=True)
    take = torch.zeros(B, N, N, dtype=torch.bool)
    ranks = torch.arange(N)[None, None, :]
    take.scatter_(2, order.indices, (ranks < k) & torch.isfinite(order.values))
    allowed = take | eye
    bias = torch.zeros(B, N, N).masked_fill(~allowed, float("-inf"))[:, None].expand(B, H, N, N).contiguous()

    with torch.no_grad():
        h = x
        for layer, blk in enumerate(blocks):
            h = blk(h, cond, pad_mask=pad, attn_head_bias=bias if layer % 2 else None)
    def checks(blk):  # per state-dict entry: float64 sum and sum of squares
        return np.array([[float(t.double().sum()), float(t.double().square().sum())]
                         for t in blk.state_dict().values()])

    np.savez_compressed(
        HERE / "trunk_alternating_b4.npz",
        x=x.numpy(), cond=cond.numpy(), coords=coords.numpy(), counts=counts.numpy(), pad_mask=pad.numpy(),
        allowed=allowed.numpy(), out=h.numpy(),
        param_checks_even=np.stack([checks(b) for b in blocks[0::2]]),
        param_checks_odd=np.stack([checks(b) for b in blocks[1::2]]),
        param_names_even=np.array(list(blocks[0].state_dict().keys())),
        param_names_odd=np.array(list(blocks[1].state_dict().keys())),
        seed=np.array(TRUNK_SEED), ada_std=np.array(TRUNK_ADA_STD), shape=np.array([B, d, H, L, k]),
    )


def geometry_bias_case(transformer, geometry) -> None:
    """SimplicialGeometryBias (transformer.py:516-996) on the reference adapter's features, by the procedure of
    tests/geometry_bias_fixture.py: the low-rank case (factorized u, v, w + angle and message factors) and the
    dense angle-residual case."""
    sys.path.insert(0, str(HERE.parent))
    import geometry_bias_fixture as fx

    coords, pad, sigma = fx.inputs()
    feats = geometry.NonPeriodicGeometryAdapter()(coords, pad_mask=pad)
    arrays = dict(coords=coords.numpy(), pad_mask=pad.numpy(), sigma=sigma.numpy(),
                  pair_delta=feats.pair_delta.numpy(), pair_dist=feats.pair_dist.numpy(),
                  pair_dist2=feats.pair_dist2.numpy(), pair_dist_norm=feats.pair_dist_norm.numpy(),
                  pair_mask=feats.pair_mask.numpy(), global_geom=feats.global_geom.numpy())
    for case in fx.CASES:
        module, result = fx.build(transformer.SimplicialGeometryBias, case, feats, pad, sigma)
        for k, v in fx.outputs(result).items():
            arrays[f"{case}_{k}"] = v
        arrays[f"{case}_param_checks"] = fx.param_checks(module)
        arrays[f"{case}_param_names"] = np.array(list(module.state_dict().keys()))
    np.savez_compressed(fx.GOLDEN, **arrays)


def main(reference_root: str) -> None:
    sys.path.insert(0, str(Path(reference_root) / "src"))
    if len(sys.argv) > 2 and sys.argv[2] == "geometry_bias":
        import matterformer.geometry.adapters as geometry  # noqa: E402
        import matterformer.models.transformer as transformer  # noqa: E402

        geometry_bias_case(transformer, geometry)
        print("wrote the geometry-bias fixture to", HERE)
        return
    if len(sys.argv) > 2 and sys.argv[2] == "trunk":
        import matterformer.geometry.adapters as geometry  # noqa: E402
        import matterformer.models.transformer as transformer  # noqa: E402

        trunk_case(transformer, geometry)
        print("wrote the trunk fixture to", HERE)
        return
    import matterformer.models.simplicial_attention as ref  # noqa: E402
    from matterformer.geometry import NonPeriodicGeometryAdapter, PeriodicGeometryAdapter  # noqa: E402
    from matterformer.geometry.lattice import lattice_latent_to_gram  # noqa: E402

    # --- 2-simplicial attention torch path ---
    _simplicial_case(ref, "fp32_padding", seed=10, B=2, H=4, N=5, D=8, dtype=torch.float32,
                     fp32_core=False, counts=[4, 2], chunk_size=2)
    _simplicial_case(ref, "fp32_holes_pairvalid", seed=11, B=3, H=2, N=9, D=16, dtype=torch.float32,
                     fp32_core=False, counts=[9, 6, 1], holes=[(0, 3), (1, 0)], pair_drop=0.3, chunk_size=4)
    _simplicial_case(ref, "fp32_qm9_slice", seed=12, B=4, H=8, N=29, D=32, dtype=torch.float32,
                     fp32_core=False, counts=[29, 17, 9, 23])
    _simplicial_case(ref, "bf16_native", seed=13, B=2, H=2, N=13, D=32, dtype=torch.bfloat16,
                     fp32_core=False, counts=[13, 7])
    _simplicial_case(ref, "bf16_fp32core", seed=14, B=2, H=2, N=13, D=32, dtype=torch.bfloat16,
                     fp32_core=True, counts=[13, 7])
    _simplicial_case(ref, "bf16_geom_slice", seed=15, B=2, H=2, N=181, D=64, dtype=torch.bfloat16,
                     fp32_core=False, counts=[57, 33])
    _simplicial_case(ref, "fp32_bias_angle_message", seed=16, B=1, H=2, N=7, D=8, dtype=torch.float32,
                     fp32_core=False, counts=[5], pair_drop=0.2, bias=True, angle_rank=5, message_rank=3,
                     chunk_size=3)

    # --- geometry conventions: pairwise distances and minimum image ---
    gen = torch.Generator().manual_seed(20)
    coords = torch.randn(3, 37, 3, generator=gen) * math.sqrt(2.0)
    pad = torch.zeros(3, 37, dtype=torch.bool)
    pad[1, 30:] = True
    feats = NonPeriodicGeometryAdapter()(coords, pad_mask=pad)
    np.savez_compressed(
        HERE / "geometry_nonperiodic.npz",
        coords=coords.numpy(), pad_mask=pad.numpy(),
        pair_dist2=feats.pair_dist2.numpy(), pair_dist=feats.pair_dist.numpy(),
    )

    gen = torch.Generator().manual_seed(21)
    ncell, nat = 3, 40
    frac = torch.rand(ncell, nat, 3, generator=gen)
    lengths = 15.0 + 15.0 * torch.rand(ncell, 3, generator=gen)
    angles = (80.0 + 20.0 * torch.rand(ncell, 3, generator=gen)) * math.pi / 180.0
    lattice = torch.cat([lengths.log(), angles.cos()], dim=-1)
    feats = PeriodicGeometryAdapter(pbc_radius=1, lattice_repr="y1")(frac, lattice=lattice)
    gram = lattice_latent_to_gram(lattice, lattice_repr="y1")
    np.savez_compressed(
        HERE / "geometry_periodic.npz",
        frac=frac.numpy(), lattice_y1=lattice.numpy(), gram=gram.numpy(),
        pair_dist2=feats.pair_dist2.numpy(), pair_delta=feats.pair_delta.numpy(),
    )
    print("wrote fixtures to", HERE)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
