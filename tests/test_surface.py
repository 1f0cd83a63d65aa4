"""The drop-in Python surface on the CPU: the product torch path, dispatch, exports, autograd plumbing.

Counterparts of the reference's own CPU tests in
tests/test_simplicial_attention.py (stases/Matterformer):

  golden vectors        the product ``simplicial_attention_torch_from_projected``
                        (matterformer_amd.simplicial_types, what ``impl="torch"``
                        runs) reproduces every fixture written from the
                        reference's torch path bit for bit
  :299-311              factorized bias summed in fp32 (KAT)
  :415-445              masked keys do not change the output (invariance)
  :448-463              a single valid pair gives v1_0 (.) v2_0 (closed form)
  :383-406              content_logits="off" equals a zero content query
  :409-412              message_mode="none" creates no message_basis
  :466-506              auto dispatch falls back to torch; explicit "triton" raises
  :509-528              compatibility re-exports
  :713-814              the 21-argument autograd Function passes the
                        needs_input_grad flags to the backward it looks up through
                        the module globals (monkeypatched here as there)
"""

from __future__ import annotations

import importlib
from pathlib import Path

import numpy as np
import pytest
import torch

import matterformer_amd.simplicial_attention as attention_module
from matterformer_amd.attention import (
    SimplicialAttention,
    SimplicialAttentionMask,
    SimplicialFactorizedBias,
    SimplicialLowRankAngleResidual,
    SimplicialLowRankMessageResidual,
    TwoSimplicialAttention,
    _TritonTwoSimplicialAttentionFunction,
    simplicial_attention_torch_from_projected,
)
from matterformer_amd.triton_regular_attention import TRITON_REGULAR_ATTENTION_AVAILABLE

GOLDEN = Path(__file__).resolve().parent / "golden"
GOLDEN_CASES = ["fp32_padding", "fp32_holes_pairvalid", "fp32_qm9_slice", "bf16_native", "bf16_fp32core",
                "bf16_geom_slice", "fp32_bias_angle_message"]


def _load_case(name):
    z = np.load(GOLDEN / f"simplicial_{name}.npz")
    dtype = getattr(torch, str(z["dtype"]))
    t = {k: torch.from_numpy(z[k]) for k in z.files if z[k].dtype != np.dtype("<U1") and z[k].ndim > 0}
    ops = [t[k].to(dtype) for k in ("q", "k1", "v1", "k2", "v2")]
    mask = SimplicialAttentionMask(query_valid=t["query_valid"], pair_key_valid=t["pair_key_valid"],
                                   pair_valid=t.get("pair_valid"))
    fb = ar = mr = basis = None
    if "u" in t:
        fb = SimplicialFactorizedBias(u=t["u"].to(dtype), v=t["v_bias"].to(dtype), w=t["w"].to(dtype),
                                      gate=t["gate"].to(dtype))
    if "angle_left" in t:
        ar = SimplicialLowRankAngleResidual(left=t["angle_left"].to(dtype), right=t["angle_right"].to(dtype),
                                            gate=t["angle_gate"].to(dtype))
    if "message_left" in t:
        mr = SimplicialLowRankMessageResidual(left=t["message_left"].to(dtype), right=t["message_right"].to(dtype))
        basis = t["message_basis"].to(dtype)
    return z, dtype, ops, mask, fb, ar, mr, basis


@pytest.mark.parametrize("name", GOLDEN_CASES)
def test_product_torch_path_matches_reference_golden_bit_for_bit(name):
    z, dtype, ops, mask, fb, ar, mr, basis = _load_case(name)
    out = simplicial_attention_torch_from_projected(
        *ops, attention_mask=mask, factorized_bias=fb, angle_residual=ar, message_residual=mr,
        message_basis=basis, chunk_size=int(z["chunk_size"]), fp32_core=bool(z["fp32_core"]))
    assert str(out.dtype).replace("torch.", "") == str(z["out_dtype"])
    assert torch.equal(out.float(), torch.from_numpy(z["out"])), name


def test_factorized_bias_chunk_sums_in_fp32():
    u = torch.full((1, 1, 2, 2), 1.0, dtype=torch.bfloat16)
    v = torch.full((1, 1, 2, 2), 0.00390625, dtype=torch.bfloat16)
    w = torch.full((1, 1, 2, 2), 0.00390625, dtype=torch.bfloat16)
    gate = torch.ones((1, 1, 2), dtype=torch.bfloat16)
    chunk = SimplicialFactorizedBias(u=u, v=v, w=w, gate=gate).chunk(0, 2, dtype=torch.float32, device=u.device)
    fp32_sum = u.float()[..., :, None] + v.float()[..., None, :] + w.float()[:, :, None]
    native = (u[..., :, None] + v[..., None, :] + w[:, :, None]).float()
    assert torch.allclose(chunk, fp32_sum)
    assert not torch.allclose(chunk, native)


def test_masked_keys_do_not_change_the_output():
    gen = torch.Generator().manual_seed(0)
    q, k1, v1, k2, v2 = (torch.randn(1, 1, 3, 4, generator=gen) for _ in range(5))
    mask = SimplicialAttentionMask(query_valid=torch.tensor([[True, True, True]]),
                                   pair_key_valid=torch.tensor([[True, True, False]]))
    out = simplicial_attention_torch_from_projected(q, k1, v1, k2, v2, attention_mask=mask, chunk_size=3)
    alt = [t.clone() for t in (k1, v1, k2, v2)]
    for t, val in zip(alt, (1000.0, -1000.0, 2000.0, 3000.0)):
        t[:, :, 2] = val
    out_alt = simplicial_attention_torch_from_projected(q, alt[0], alt[1], alt[2], alt[3], attention_mask=mask,
                                                        chunk_size=3)
    assert torch.allclose(out, out_alt, atol=1e-6, rtol=1e-5)


def test_single_valid_pair_closed_form():
    z = torch.zeros(1, 1, 3, 2)
    v1 = torch.tensor([[[[1.0, 2.0], [5.0, 7.0], [11.0, 13.0]]]])
    v2 = torch.tensor([[[[3.0, 5.0], [17.0, 19.0], [23.0, 29.0]]]])
    pv = torch.zeros(1, 3, 3, dtype=torch.bool)
    pv[:, 0, 0] = True
    valid = torch.ones(1, 3, dtype=torch.bool)
    mask = SimplicialAttentionMask(query_valid=valid, pair_key_valid=valid, pair_valid=pv)
    out = simplicial_attention_torch_from_projected(z, z, v1, z, v2, attention_mask=mask, chunk_size=3)
    assert torch.allclose(out, torch.tensor([3.0, 10.0]).view(1, 1, 1, 2).expand_as(out), atol=1e-6)


def test_content_logits_off_matches_zero_content_query():
    torch.manual_seed(0)
    attn = TwoSimplicialAttention(dim=32, num_heads=4, impl="torch", chunk_size=3, content_logits="off")
    x = torch.randn(2, 5, 32)
    kpm = torch.tensor([[False, False, False, False, True], [False, False, True, True, True]])
    q, k1, v1, k2, v2 = attn._project_inputs(x)
    mask = SimplicialAttentionMask.from_key_padding_mask(kpm, batch_size=2, num_tokens=5, device=x.device)
    heads = simplicial_attention_torch_from_projected(torch.zeros_like(q), k1, v1, k2, v2, attention_mask=mask,
                                                      chunk_size=attn.chunk_size)
    assert torch.allclose(attn(x, key_padding_mask=kpm), attn.out_proj(attn._merge_heads(heads)),
                          atol=1e-6, rtol=1e-5)


def test_message_mode_none_creates_no_message_basis():
    attn = TwoSimplicialAttention(dim=32, num_heads=4, message_mode="none")
    assert attn.message_basis is None
    assert "message_basis" not in dict(attn.named_parameters())


def test_constructor_validation_errors():
    with pytest.raises(ValueError, match="must be divisible"):
        SimplicialAttention(dim=30, num_heads=4)
    with pytest.raises(ValueError, match="Unsupported simplicial_impl"):
        SimplicialAttention(dim=32, num_heads=4, impl="cuda")
    with pytest.raises(ValueError, match="Unsupported simplicial_precision"):
        SimplicialAttention(dim=32, num_heads=4, precision="fp8")
    with pytest.raises(ValueError, match="Unsupported simplicial_message_mode"):
        SimplicialAttention(dim=32, num_heads=4, message_mode="dense")
    with pytest.raises(ValueError, match="simplicial_content_logits"):
        SimplicialAttention(dim=32, num_heads=4, content_logits="maybe")
    assert SimplicialAttention(dim=32, num_heads=4, impl="hip").impl == "triton"


def test_auto_dispatch_falls_back_to_torch_for_cpu_and_unsupported_modes():
    torch.manual_seed(0)
    x = torch.randn(2, 4, 32)
    kpm = torch.tensor([[False, False, False, True], [False, False, True, True]])

    auto = TwoSimplicialAttention(dim=32, num_heads=4, impl="auto")
    auto(x, key_padding_mask=kpm)
    assert auto._last_impl_used == "torch"
    reason = auto._triton_unavailable_reason(x=x, factorized_bias=None, angle_residual=None, message_residual=None,
                                             message_basis=None, logit_bias_fn=None, return_attn=False)
    assert reason is not None

    dropout = TwoSimplicialAttention(dim=32, num_heads=4, impl="auto", dropout=0.1)
    dropout.train()
    dropout(x, key_padding_mask=kpm)
    assert dropout._last_impl_used == "torch"

    with_fn = TwoSimplicialAttention(dim=32, num_heads=4, impl="auto")

    def residual(start, end, dtype, device):
        return torch.zeros(x.shape[0], 4, end - start, x.shape[1], x.shape[1], dtype=dtype, device=device)

    with_fn(x, key_padding_mask=kpm, logit_bias_fn=residual)
    assert with_fn._last_impl_used == "torch"

    _, attn = auto(x, key_padding_mask=kpm, return_attn=True)
    assert auto._last_impl_used == "torch"
    assert attn.shape == (2, 4, 4, 4, 4)

    explicit = TwoSimplicialAttention(dim=32, num_heads=4, impl="triton")
    with pytest.raises(RuntimeError, match="unavailable"):
        explicit(x, key_padding_mask=kpm)


def test_compatibility_re_exports_retained_names():
    compat = importlib.import_module("matterformer_amd.attention")
    triton_mod = importlib.import_module("matterformer_amd.attention_triton")
    launcher = importlib.import_module("matterformer_amd.hip_simplicial_attention")
    # the export lists of src/matterformer/models/attention.py:22-37 and attention_triton.py:12-19
    assert set(compat.__all__) == {
        "TRITON_AVAILABLE", "SUPPORTED_SIMPLICIAL_PRECISIONS", "SimplicialAttention", "SimplicialAttentionMask",
        "SimplicialFactorizedBias", "SimplicialLowRankAngleResidual", "SimplicialLowRankMessageResidual",
        "TwoSimplicialAttention", "_TritonTwoSimplicialAttentionFunction", "normalize_simplicial_precision",
        "simplicial_attention_torch_from_projected", "triton_block_d_for_head_dim",
        "triton_simplicial_attention_backward", "triton_simplicial_attention_forward",
    }
    assert set(triton_mod.__all__) == {
        "TRITON_AVAILABLE", "SUPPORTED_SIMPLICIAL_PRECISIONS", "normalize_simplicial_precision",
        "triton_block_d_for_head_dim", "triton_simplicial_attention_backward",
        "triton_simplicial_attention_forward",
    }
    for name in compat.__all__:
        assert hasattr(compat, name), name
    assert compat.SimplicialAttention is SimplicialAttention
    assert compat.TwoSimplicialAttention is SimplicialAttention
    assert triton_mod.triton_simplicial_attention_forward is launcher.hip_simplicial_attention_forward
    assert triton_mod.triton_simplicial_attention_backward is launcher.hip_simplicial_attention_backward
    assert launcher.SUPPORTED_SIMPLICIAL_PRECISIONS == ("bf16_tc", "tf32", "ieee_fp32")
    assert [launcher.triton_block_d_for_head_dim(d) for d in (1, 16, 17, 33, 64, 100, 128)] == \
        [16, 16, 32, 64, 64, 128, 128]
    with pytest.raises(ValueError):
        launcher.triton_block_d_for_head_dim(129)
    assert launcher.normalize_simplicial_precision("BF16_TC") == "bf16_tc"
    assert TRITON_REGULAR_ATTENTION_AVAILABLE is False


def test_autograd_function_passes_optional_gradient_flags(monkeypatch):
    captured: dict[str, bool] = {}

    def fake_forward(q, k1, v1, k2, v2, **kwargs):
        out = torch.zeros_like(q)
        return out, q.new_zeros(q.shape[:3], dtype=torch.float32), out.float()

    def fake_backward(grad_out, q, k1, v1, k2, v2, *args, **kwargs):
        for name in ("need_du", "need_dv_bias", "need_dw", "need_dgate", "need_dangle_left", "need_dangle_right",
                     "need_dangle_gate", "need_dmessage_left", "need_dmessage_right", "need_dmessage_basis"):
            captured[name] = bool(kwargs[name])
        zeros = [torch.zeros_like(t) for t in (q, k1, v1, k2, v2)]
        return (*zeros, None, None, None, None, torch.zeros_like(kwargs["angle_left"]), None,
                torch.zeros_like(kwargs["angle_gate"]), None, torch.zeros_like(kwargs["message_right"]), None)

    monkeypatch.setattr(attention_module, "triton_simplicial_attention_forward", fake_forward)
    monkeypatch.setattr(attention_module, "triton_simplicial_attention_backward", fake_backward)

    q = torch.randn(1, 2, 3, 4, requires_grad=True)
    k1, v1, k2, v2 = (torch.randn_like(q, requires_grad=True) for _ in range(4))
    ones = torch.ones(1, 3, dtype=torch.bool)
    u = torch.randn(1, 2, 3, 3)
    angle_left = torch.randn(1, 2, 3, 3, 2, requires_grad=True)
    angle_gate = torch.randn(1, 2, 3, requires_grad=True)
    message_right = torch.randn(1, 2, 3, 3, 2, requires_grad=True)
    out = _TritonTwoSimplicialAttentionFunction.apply(
        q, k1, v1, k2, v2, ones, ones, torch.empty(0, dtype=torch.bool),
        u, torch.randn_like(u), torch.randn_like(u), torch.randn(1, 2, 3),
        angle_left, torch.randn(1, 2, 3, 3, 2), angle_gate,
        torch.randn(1, 2, 3, 3, 2), message_right, torch.randn(2, 2, 4),
        "ieee_fp32", 128, False)
    out.sum().backward()
    assert captured == {
        "need_du": False, "need_dv_bias": False, "need_dw": False, "need_dgate": False,
        "need_dangle_left": True, "need_dangle_right": False, "need_dangle_gate": True,
        "need_dmessage_left": False, "need_dmessage_right": True, "need_dmessage_basis": False,
    }
    assert q.grad is not None and torch.count_nonzero(q.grad) == 0


def test_debug_torch_backward_recompute_matches_autograd_of_torch_path():
    """debug_torch_backward=True (simplicial_attention.py:454-552) recomputes with the fp32-core torch path;
    with a forward swapped in for the kernel this runs on the CPU and must equal plain autograd."""
    gen = torch.Generator().manual_seed(3)
    B, H, N, D = 1, 2, 6, 8
    base = [torch.randn(B, H, N, D, generator=gen) for _ in range(5)]
    qv = torch.ones(B, N, dtype=torch.bool)
    pkv = qv.clone()
    pkv[0, 5] = False
    fbt = [torch.randn(B, H, N, N, generator=gen) for _ in range(3)] + [torch.randn(B, H, N, generator=gen)]
    mask = SimplicialAttentionMask(query_valid=qv, pair_key_valid=pkv)

    def torch_forward(q, k1, v1, k2, v2, **kw):
        fb = SimplicialFactorizedBias(u=kw["u"], v=kw["v_bias"], w=kw["w"], gate=kw["gate"])
        m = SimplicialAttentionMask(query_valid=kw["query_valid"], pair_key_valid=kw["pair_key_valid"])
        o = simplicial_attention_torch_from_projected(q, k1, v1, k2, v2, attention_mask=m, factorized_bias=fb,
                                                      fp32_core=True)
        return o.to(q.dtype), q.new_zeros(q.shape[:3]), o

    leaves = [t.clone().requires_grad_(True) for t in base + fbt]
    with pytest.MonkeyPatch.context() as mp:
        mp.setattr(attention_module, "triton_simplicial_attention_forward", torch_forward)
        out = _TritonTwoSimplicialAttentionFunction.apply(
            *leaves[:5], qv, pkv, torch.empty(0, dtype=torch.bool), *leaves[5:],
            *(torch.empty(0) for _ in range(6)), "ieee_fp32", 4, True)
    (out.square().mean()).backward()
    ref = [t.clone().requires_grad_(True) for t in base + fbt]
    fb = SimplicialFactorizedBias(u=ref[5], v=ref[6], w=ref[7], gate=ref[8])
    expected = simplicial_attention_torch_from_projected(*ref[:5], attention_mask=mask, factorized_bias=fb,
                                                         chunk_size=4, fp32_core=True)
    expected.square().mean().backward()
    for got, exp in zip(leaves, ref):
        assert torch.allclose(got.grad, exp.grad, atol=1e-6, rtol=1e-5)
