"""Host-side proof that mf_geometry_features stays inside its buffers.

The launch of csrc/geometry.hip is replayed on the CPU: every (workgroup,
wave, grid-stride iteration, lane) of ``features_kernel<R>`` and every thread
of ``rms_kernel`` is enumerated with numpy, each global read and write index
the kernel forms is computed from the same integer expressions, and the test
asserts that every index lies inside the buffer the adapter allocates
(``geometry.py`` ``_hip_features``: delta (B, N, N, 3), d2 / d / d_norm
(B, N, N) fp32, pair mask (B, N, N) u8, bits (B, N, ceil(N/32)) i32, scale
(B,)) and that every output element is written exactly once (so no
``torch.empty`` byte survives).  The index arithmetic does not depend on R
(the number of images only changes register work), so one replay covers
``features_kernel<0|1|2>``; the shapes include configs[3] (8 cells x 512
atoms, 27 images, 6 A cutoff bits) and ragged ones.
"""
from __future__ import annotations

import numpy as np
import pytest

WAVES_PER_BLOCK = 4  # kThreads / 64 in geometry.hip
THREADS = 256


def _launch_grid(B: int, N: int, num_cus: int) -> int:
    """The launcher's grid: min(ceil(units / 4), num_cus * 32)."""
    chunks = (N + 63) // 64
    units = B * N * chunks
    return min((units + WAVES_PER_BLOCK - 1) // WAVES_PER_BLOCK, num_cus * 32)


def _replay_features(B: int, N: int, *, pad: bool, bits: bool, num_cus: int) -> dict[str, np.ndarray]:
    """Every index features_kernel forms, one entry per (unit, lane) access that executes."""
    W = (N + 31) // 32
    chunks = (N + 63) // 64
    units = B * N * chunks
    grid = _launch_grid(B, N, num_cus)
    # the grid-stride loop: wave gw = blockIdx * 4 + wave takes u = gw, gw + grid * 4, ... while u < units
    gw = np.arange(grid * WAVES_PER_BLOCK, dtype=np.int64)
    stride = grid * WAVES_PER_BLOCK
    iters = -(-units // stride)
    u = (gw[None, :] + stride * np.arange(iters, dtype=np.int64)[:, None]).ravel()
    u = u[u < units]
    lane = np.arange(64, dtype=np.int64)
    chunk = (u % chunks)[:, None]
    row = (u // chunks)[:, None]
    b = row // N
    j = chunk * 64 + lane[None, :]
    in_row = j < N
    full = np.ones_like(j, dtype=bool)
    acc: dict[str, tuple[np.ndarray, np.ndarray]] = {}
    acc["units"] = (u, np.ones_like(u, dtype=bool))
    if pad:
        acc["pad_i"] = (np.broadcast_to(row, j.shape), full)
        acc["pad_j"] = (b * N + j, in_row)          # read only where j < N (short-circuit)
    jj = np.where(in_row, j, 0)
    for c in range(3):
        acc[f"coords_i{c}"] = (np.broadcast_to(row * 3 + c, j.shape), full)
        acc[f"coords_j{c}"] = ((b * N + jj) * 3 + c, full)
        acc[f"gram{c}"] = (np.broadcast_to(b * 9 + 3 * c, j.shape), full)
        acc[f"gram{c}_last"] = (np.broadcast_to(b * 9 + 3 * c + 2, j.shape), full)
    o = row * N + j
    for c in range(3):
        acc[f"delta{c}"] = (3 * o + c, in_row)
    acc["o"] = (o, in_row)
    acc["scale"] = (np.broadcast_to(b, j.shape), in_row)
    if bits:
        w = 2 * chunk + (lane[None, :] >> 5)
        writer = ((lane[None, :] & 31) == 0) & (w < W)
        acc["bits"] = (row * W + w, writer)
    return {k: idx[np.broadcast_to(m, idx.shape)] for k, (idx, m) in acc.items()}


CASES = [
    # (B, N, pad, bits, num_cus)
    (8, 512, True, True, 256),    # configs[3]: the periodic cells with the cutoff bits, MI355X CU count
    (8, 512, False, True, 256),
    (8, 512, True, True, 3),      # few CUs: several grid-stride iterations per wave
    (3, 500, True, True, 256),    # ragged: the last chunk's upper half-wave has no bits word
    (2, 33, True, True, 256),
    (1, 1, False, True, 256),
    (4, 96, True, True, 7),       # N = 32 mod 64: the last half-wave's bits word would be word W
    (4, 96, True, False, 7),
]


@pytest.mark.parametrize("B,N,pad,bits,num_cus", CASES)
def test_features_kernel_indices_stay_in_bounds(B, N, pad, bits, num_cus):
    W = (N + 31) // 32
    acc = _replay_features(B, N, pad=pad, bits=bits, num_cus=num_cus)
    sizes = {"pad": B * N, "coords": 3 * B * N, "gram": 9 * B, "delta": 3 * B * N * N, "o": B * N * N,
             "scale": B, "bits": B * N * W}

    def check(name: str, size: int) -> None:
        idx = acc[name]
        assert idx.size == 0 or (idx.min() >= 0 and idx.max() < size), (name, idx.min(), idx.max(), size)

    # every unit is visited exactly once by the grid-stride loop
    assert np.array_equal(np.sort(acc["units"]), np.arange(B * N * ((N + 63) // 64)))
    if pad:
        check("pad_i", sizes["pad"])
        check("pad_j", sizes["pad"])
    for c in range(3):
        check(f"coords_i{c}", sizes["coords"])
        check(f"coords_j{c}", sizes["coords"])
        check(f"gram{c}", sizes["gram"])
        check(f"gram{c}_last", sizes["gram"])
        check(f"delta{c}", sizes["delta"])
    check("o", sizes["o"])
    check("scale", sizes["scale"])
    # each output element is written once: no stale torch.empty byte and no double write
    o = acc["o"]
    assert o.size == B * N * N and np.unique(o).size == o.size
    d = np.concatenate([acc[f"delta{c}"] for c in range(3)])
    assert np.unique(d).size == d.size == 3 * B * N * N
    if bits:
        check("bits", sizes["bits"])
        w = acc["bits"]
        assert w.size == B * N * W and np.unique(w).size == w.size


@pytest.mark.parametrize("B,N", [(8, 512), (64, 29), (3, 257)])
def test_rms_kernel_indices_stay_in_bounds(B, N):
    """rms_kernel: one workgroup per molecule, thread a reads atoms a, a + 256, ... < N; thread 0 writes scale[b]."""
    b = np.arange(B, dtype=np.int64)[:, None, None]
    tid = np.arange(THREADS, dtype=np.int64)[None, :, None]
    steps = np.arange(-(-N // THREADS), dtype=np.int64)[None, None, :]
    a = tid + THREADS * steps
    live = np.broadcast_to(a < N, (B, THREADS, steps.shape[-1]))
    r = np.broadcast_to(b * N + a, live.shape)[live]
    assert r.min() >= 0 and r.max() < B * N                 # pad[r]
    assert (3 * r + 2).max() < 3 * B * N                    # coords[3 r + 2]
    assert np.unique(r).size == B * N                       # every atom read once per molecule
    assert b.max() < B                                      # scale[b]


def test_launch_grid_matches_units_at_config4():
    """configs[3] on 256 CUs: 8 x 512 rows x 8 chunks = 32768 units, 8192 workgroups, one unit per wave."""
    assert _launch_grid(8, 512, 256) == 8192
