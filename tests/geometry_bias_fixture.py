"""Shared by tests/golden/make_golden.py (reference module) and the geometry-bias tests (mirrored module): the
same seeded construction, first call and parameter overwrite for SimplicialGeometryBias, so both draw the same
weights and their outputs can be compared.

Procedure: torch.manual_seed(SEED); construct with the case's keyword arguments; one
build_structured_bias_inputs call (materialises the LazyLinear layers in the module's call order; the dense
angle-residual case also calls its callback once); then every parameter that is all zeros (the zero-initialised
output layers, the noise-gate beta) is overwritten with N(0, 0.3^2) draws from torch.Generator(SEED + 100),
in named_parameters order; the second call's outputs are the fixture.
"""

from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden" / "geometry_bias.npz"
SEED = 31
B, N, H, HIDDEN = 3, 11, 4, 32
CASES = {
    "lowrank": dict(mode="angle_low_rank", message_mode="low_rank", angle_residual_rank=3, message_rank=2,
                    edge_bias_hidden_dim=HIDDEN),
    "residual": dict(mode="angle_residual", edge_bias_hidden_dim=HIDDEN),
}


def inputs():
    gen = torch.Generator().manual_seed(SEED)
    coords = torch.randn(B, N, 3, generator=gen) * 1.3
    pad = torch.zeros(B, N, dtype=torch.bool)
    pad[1, 8:] = True
    pad[2, 5:] = True
    sigma = torch.rand(B, generator=gen) * 2.0 + 0.05
    return coords, pad, sigma


def build(module_cls, case: str, features, pad, sigma):
    torch.manual_seed(SEED)
    m = module_cls(H, **CASES[case])
    first = m.build_structured_bias_inputs(features, coords_len=N, pad_mask=pad, sigma=sigma)
    if first[1] is not None:
        first[1](0, N, torch.float32, torch.device("cpu"))
    gen = torch.Generator().manual_seed(SEED + 100)
    with torch.no_grad():
        for _, prm in m.named_parameters():
            if not prm.any():
                prm.copy_(torch.randn(prm.shape, generator=gen) * 0.3)
    return m, m.build_structured_bias_inputs(features, coords_len=N, pad_mask=pad, sigma=sigma)


def outputs(result) -> dict:
    fb, residual_fn, angle, message, mask = result
    out = {"u": fb.u, "v": fb.v, "w": fb.w, "gate": fb.gate, "query_valid": mask.query_valid,
           "pair_key_valid": mask.pair_key_valid, "pair_valid": mask.pair_valid}
    if angle is not None:
        out.update(angle_left=angle.left, angle_right=angle.right, angle_gate=angle.gate)
    if message is not None:
        out.update(message_left=message.left, message_right=message.right)
    if residual_fn is not None:
        out["residual"] = residual_fn(0, N, torch.float32, torch.device("cpu"))
    return {k: v.detach().cpu().numpy() for k, v in out.items()}


def param_checks(m) -> np.ndarray:
    return np.array([[float(t.double().sum()), float(t.double().square().sum())] for t in m.state_dict().values()])
