"""Build + ctypes wrappers of the oracle's C restatements (TEST INFRASTRUCTURE ONLY).

``build()`` compiles oracle/*.c with gcc (-O2 -ffp-contract=off, no fast math)
into oracle/_build/liboracle.so.  The reference itself is pure Python, so there
is no reference C code to build under oracle/_ref.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
BUILD_DIR = HERE / "_build"
LIB_PATH = BUILD_DIR / "liboracle.so"
SOURCES = ("knn.c", "radius.c")
CFLAGS = ["-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-Wall"]

_lib = None


def build() -> Path:
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = ["gcc", *CFLAGS, *(str(HERE / s) for s in SOURCES), "-lm", "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{proc.stderr}")
    tmp.replace(LIB_PATH)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        stale = not LIB_PATH.exists() or any(
            (HERE / s).stat().st_mtime > LIB_PATH.stat().st_mtime for s in SOURCES)
        if stale:
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        i32 = ctypes.c_int32
        _lib.oracle_knn.argtypes = [P, P, i32, i32, i32, i32, P, P, P]
        _lib.oracle_knn.restype = None
        _lib.oracle_radius_mask.argtypes = [P, P, P, i32, i32, ctypes.c_float, i32, i32, P, P]
        _lib.oracle_radius_mask.restype = None
        _lib.oracle_pair_d2_matrix.argtypes = [P, P, i32, i32, i32, P]
        _lib.oracle_pair_d2_matrix.restype = None
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def knn(coords: np.ndarray, k: int, pad_mask: np.ndarray | None = None, exclude_self: bool = True):
    """coords (B,N,3) fp32 -> (idx int32 (B,N,k), dist fp32 (B,N,k))."""
    coords = np.ascontiguousarray(coords, dtype=np.float32)
    B, N, _ = coords.shape
    pad = None if pad_mask is None else np.ascontiguousarray(pad_mask, dtype=np.uint8)
    idx = np.empty((B, N, k), dtype=np.int32)
    dist = np.empty((B, N, k), dtype=np.float32)
    scratch = np.empty(N, dtype=np.float32)
    lib().oracle_knn(_p(coords), _p(pad), B, N, k, int(exclude_self), _p(idx), _p(dist), _p(scratch))
    return idx, dist


def radius_mask(coords: np.ndarray, cutoff: float, gram: np.ndarray | None = None,
                pad_mask: np.ndarray | None = None, pbc_radius: int = 1, block: int = 64):
    """-> (bits uint32 (B,N,ceil(N/32)), block_mask uint8 (B,NB,NB))."""
    coords = np.ascontiguousarray(coords, dtype=np.float32)
    B, N, _ = coords.shape
    g = None if gram is None else np.ascontiguousarray(gram, dtype=np.float32)
    pad = None if pad_mask is None else np.ascontiguousarray(pad_mask, dtype=np.uint8)
    W = (N + 31) // 32
    NB = (N + block - 1) // block
    bits = np.empty((B, N, W), dtype=np.uint32)
    blocks = np.empty((B, NB, NB), dtype=np.uint8)
    lib().oracle_radius_mask(_p(coords), _p(g), _p(pad), B, N, float(cutoff), pbc_radius, block, _p(bits),
                             _p(blocks))
    return bits, blocks


def pair_d2(coords: np.ndarray, gram: np.ndarray | None = None, pbc_radius: int = 1) -> np.ndarray:
    coords = np.ascontiguousarray(coords, dtype=np.float32)
    B, N, _ = coords.shape
    g = None if gram is None else np.ascontiguousarray(gram, dtype=np.float32)
    out = np.empty((B, N, N), dtype=np.float32)
    lib().oracle_pair_d2_matrix(_p(coords), _p(g), B, N, pbc_radius, _p(out))
    return out


def unpack_bits(bits: np.ndarray, N: int) -> np.ndarray:
    """(B,R,W) uint32 -> (B,R,N) bool (bit t of word w is column 32 w + t)."""
    B, R, W = bits.shape
    shifts = np.arange(32, dtype=np.uint32)
    full = ((bits[..., None] >> shifts) & 1).astype(bool).reshape(B, R, W * 32)
    return full[..., :N]
