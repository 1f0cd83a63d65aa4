"""mf_adaln_rows, mf_rows_to_heads and mf_heads_to_rows (the packed trunk's per-token glue) against the
torch expressions they replace (TokenPacking's and adaln_rows' CPU paths, transformer.py:296-316).

Bars: the two reshapes bit for bit (data movement, q's scale rounded in the source dtype as torch rounds
q * scale); mf_adaln_rows within one rounding step of the activation dtype per element, since its LayerNorm
statistics are summed in another order than torch's (an ulp of the product LN(x) * (1 + scale) and of the
result, fp32 or bf16; bf16 on at most 0.5 % of elements)."""

import pytest
import torch

from matterformer_amd.token_packing import TokenPacking, adaln_rows

pytestmark = pytest.mark.gpu


def _packing(cuda, B, N, frac, seed):
    gen = torch.Generator().manual_seed(seed)
    pad = torch.rand(B, N, generator=gen) < frac
    pad[:, 0] = False
    return TokenPacking(pad.to(cuda)), TokenPacking(pad), gen


@pytest.mark.parametrize("src,dst", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.bfloat16),
                                     (torch.float32, torch.float32), (torch.float16, torch.float16)])
@pytest.mark.parametrize("B,N,H,D,parts", [(5, 37, 8, 64, 5), (3, 181, 4, 32, 3), (2, 9, 2, 128, 1)])
def test_rows_heads_round_trip_matches_torch(cuda, src, dst, B, N, H, D, parts):
    pg, pc, gen = _packing(cuda, B, N, 0.5, B * N + D)
    proj = torch.randn(pc.tokens, parts * H * D, generator=gen).to(src)
    with torch.no_grad():
        got = pg.to_heads(proj.to(cuda), parts, H, D, dst, first_part_scale=D ** -0.5)
    want = pc.to_heads(proj, parts, H, D, dst, first_part_scale=D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(got.cpu(), want)
    for part in range(parts):
        with torch.no_grad():
            rows = pg.from_heads(got[part], src)
        assert torch.equal(rows.cpu(), pc.from_heads(want[part], src))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("C", [512, 64, 2048])
def test_adaln_rows_matches_torch(cuda, dtype, C):
    pg, pc, gen = _packing(cuda, 6, 50, 0.4, C)
    T = pc.tokens
    x = torch.randn(T, C, generator=gen).to(dtype)
    y = torch.randn(T, C, generator=gen).to(dtype)
    mods = (torch.randn(6, 6 * C, generator=gen) * 0.3).to(dtype)
    g, sh, sc = mods[:, 2 * C:3 * C], mods[:, 3 * C:4 * C], mods[:, 4 * C:5 * C]
    want_x, want_h = adaln_rows(pc, x, y, gate=g, shift=sh, scale=sc, eps=1e-6)
    want_h0 = adaln_rows(pc, x, shift=sh, scale=sc, eps=1e-6)
    mg = mods.to(cuda)
    with torch.no_grad():
        got_x, got_h = adaln_rows(pg, x.to(cuda), y.to(cuda), gate=mg[:, 2 * C:3 * C], shift=mg[:, 3 * C:4 * C],
                                  scale=mg[:, 4 * C:5 * C], eps=1e-6)
        got_h0 = adaln_rows(pg, x.to(cuda), shift=mg[:, 3 * C:4 * C], scale=mg[:, 4 * C:5 * C], eps=1e-6)
        xi = x.to(cuda)
        same = adaln_rows(pg, xi, y.to(cuda), gate=mg[:, 2 * C:3 * C], inplace=True)
    torch.cuda.synchronize()
    assert torch.equal(got_x.cpu(), want_x)  # residual: no reduction, bit for bit
    assert same.data_ptr() == xi.data_ptr() and torch.equal(xi.cpu(), want_x)
    xr = want_x.float()
    for got, want, src in ((got_h, want_h, xr), (got_h0, want_h0, x.float())):
        got = got.cpu().float()
        want = want.float()
        # one rounding of the normalised value and of the product, then the sum's own rounding: when the
        # shift nearly cancels the product the result's ulp is far below the product's
        n = torch.nn.functional.layer_norm(src, (C,), eps=1e-6)
        prod = (n * pc.per_token(1.0 + sc.float())).abs()
        if dtype == torch.float32:
            # the statistics' rounding moves LN(x) by ~1e-8 absolute, also where LN(x) is near 0
            assert bool(((got - want).abs() <= 4e-6 * (prod + want.abs()) + 1e-6).all())
        else:
            diff = (got - want).abs()
            bound = 2.0 ** -7 * (2.0 * prod + want.abs())
            assert bool((diff <= bound + 1e-30).all())
            assert float((diff > 0).float().mean()) <= 5e-3


def test_adaln_rows_rejects_bad_arguments(cuda):
    from matterformer_amd import _native

    lib = _native.lib()
    args = _native.MfAdalnRowsArgs(tokens=1, channels=12, batch=1, mod_stride=12, dtype=0, eps=1e-6)
    assert lib.mf_adaln_rows(args, None) == -1  # x and mol NULL
    x = torch.zeros(1, 12, device=cuda)
    mol = torch.zeros(1, dtype=torch.int32, device=cuda)
    args = _native.MfAdalnRowsArgs(x=x.data_ptr(), mol=mol.data_ptr(), shift=x.data_ptr(), scale=x.data_ptr(),
                                   h_out=x.data_ptr(), tokens=1, channels=12, batch=1, mod_stride=12, dtype=0,
                                   eps=1e-6)
    assert lib.mf_adaln_rows(args, None) == -2  # channels not a multiple of 8
    assert "multiples of 8" in _native.last_error()


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 1e-2)])
def test_mlp_fused_gelu_is_the_tanh_gelu(cuda, dtype, tol):
    """Mlp on packed rows without autograd folds the tanh GELU into fc1's GEMM epilogue; the result is the
    module's own fc1 -> GELU(tanh) -> fc2 (transformer.py:129-148) to the GEMM's rounding, and measurably
    farther from the erf GELU."""
    from matterformer_amd.trunk import Mlp

    torch.manual_seed(0)
    mlp = Mlp(256).to(cuda).to(dtype).eval()
    x = torch.randn(300, 256, device=cuda, dtype=dtype)
    with torch.no_grad():
        assert mlp._fused_gelu_ok(x)
        got = mlp(x).float()
        ref = mlp.fc2(torch.nn.functional.gelu(mlp.fc1(x.float() if dtype == torch.float32 else x),
                                                approximate="tanh")).float()
        erf = mlp.fc2(torch.nn.functional.gelu(mlp.fc1(x))).float()
    torch.cuda.synchronize()
    rel = float((got - ref).norm() / ref.norm())
    assert rel <= tol, rel
    if dtype == torch.float32:
        assert float((got - erf).norm() / erf.norm()) > 10 * rel
    assert not mlp._fused_gelu_ok(x.requires_grad_())
