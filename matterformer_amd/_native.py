"""ctypes binding of libmf_hip.so (the C ABI declared in include/mf_capi.h).

The library links ``libamdhip64.so.7``.  torch's ROCm build ships a HIP runtime
with the same SONAME, so importing torch (which loads it) before ``dlopen`` of
libmf_hip.so makes both share one runtime: torch's stream handles and device
pointers are then valid inside the library.

This module never falls back to another implementation: when the library is
missing, every call raises ``RuntimeError`` naming what is missing.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library must share)

from matterformer_amd.build import LIB_PATH

MF_OK = 0
MF_ERR_INVALID_ARGUMENT = -1
MF_ERR_UNSUPPORTED = -2
MF_ERR_HIP = -3

MF_DTYPE_F32 = 0
MF_DTYPE_F16 = 1
MF_DTYPE_BF16 = 2

MF_PREC = {"bf16_tc": 0, "tf32": 1, "ieee_fp32": 2}

# Every symbol include/mf_capi.h declares (tests check the library exports them).
EXPORTED_SYMBOLS = (
    "mf_abi_version",
    "mf_last_error",
    "mf_simplicial_fwd",
    "mf_simplicial_fwd_supported",
    "mf_simplicial_fwd_workspace_size",
    "mf_simplicial_fwd_noalloc",
    "mf_simplicial_bwd",
    "mf_simplicial_bwd_workspace_size",
    "mf_knn",
    "mf_knn_mask",
    "mf_radius_mask",
    "mf_geometry_features",
    "mf_radius_attn",
    "mf_adaln_rows",
    "mf_rows_to_heads",
    "mf_heads_to_rows",
    "mf_pair_mlp_bias",
    "mf_lattice_terms",
    "mf_pair_mlp_bias_bwd",
    "mf_pair_mlp_bias_bwd_workspace_size",
)

EXPECTED_ABI_VERSION = 11

_DTYPE_CODE = {
    torch.float32: MF_DTYPE_F32,
    torch.float16: MF_DTYPE_F16,
    torch.bfloat16: MF_DTYPE_BF16,
}


class MfSimplicialFwdArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k1", ctypes.c_void_p),
        ("v1", ctypes.c_void_p),
        ("k2", ctypes.c_void_p),
        ("v2", ctypes.c_void_p),
        ("query_valid", ctypes.c_void_p),
        ("pair_key_valid", ctypes.c_void_p),
        ("pair_valid", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("out_f32", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_uint64),
        ("batch", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("tokens", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("precision", ctypes.c_int32),
        ("bias_u", ctypes.c_void_p),
        ("bias_v", ctypes.c_void_p),
        ("bias_w", ctypes.c_void_p),
        ("bias_gate", ctypes.c_void_p),
        ("bias_dtype", ctypes.c_int32),
        ("angle_rank", ctypes.c_int32),
        ("angle_left", ctypes.c_void_p),
        ("angle_right", ctypes.c_void_p),
        ("angle_gate", ctypes.c_void_p),
        ("message_left", ctypes.c_void_p),
        ("message_right", ctypes.c_void_p),
        ("message_basis", ctypes.c_void_p),
        ("message_rank", ctypes.c_int32),
        ("q_stride", ctypes.c_int64 * 3),
        ("kv_stride", ctypes.c_int64 * 3),
        ("out_stride", ctypes.c_int64 * 3),
    ]


class MfSimplicialBwdArgs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "q", "k1", "v1", "k2", "v2", "grad_out", "out", "lse", "query_valid", "pair_key_valid", "pair_valid",
        "bias_u", "bias_v", "bias_w", "bias_gate")] + \
        [("bias_dtype", ctypes.c_int32), ("grad_dtype", ctypes.c_int32)] + \
        [(n, ctypes.c_void_p) for n in ("dq", "dk1", "dv1", "dk2", "dv2", "du", "dv_bias", "dw", "dgate")] + \
        [(n, ctypes.c_int32) for n in ("batch", "heads", "tokens", "head_dim", "dtype", "grads_dtype",
                                       "angle_rank", "message_rank")] + \
        [(n, ctypes.c_void_p) for n in (
            "angle_left", "angle_right", "angle_gate", "message_left", "message_right", "message_basis",
            "dangle_left", "dangle_right", "dangle_gate", "dmessage_left", "dmessage_right", "dmessage_basis",
            "workspace")] + [("workspace_bytes", ctypes.c_uint64)]


class MfKnnArgs(ctypes.Structure):
    _fields_ = [
        ("coords", ctypes.c_void_p),
        ("pad_mask", ctypes.c_void_p),
        ("idx", ctypes.c_void_p),
        ("dist", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("atoms", ctypes.c_int32),
        ("k", ctypes.c_int32),
        ("exclude_self", ctypes.c_int32),
    ]


class MfKnnMaskArgs(ctypes.Structure):
    _fields_ = [
        ("idx", ctypes.c_void_p),
        ("pad_mask", ctypes.c_void_p),
        ("mask_bits", ctypes.c_void_p),
        ("block_mask", ctypes.c_void_p),
        ("batch", ctypes.c_int32),
        ("atoms", ctypes.c_int32),
        ("k", ctypes.c_int32),
        ("include_self", ctypes.c_int32),
    ]


class MfRadiusMaskArgs(ctypes.Structure):
    _fields_ = [
        ("coords", ctypes.c_void_p),
        ("gram", ctypes.c_void_p),
        ("pad_mask", ctypes.c_void_p),
        ("mask_bits", ctypes.c_void_p),
        ("block_mask", ctypes.c_void_p),
        ("cutoff", ctypes.c_float),
        ("batch", ctypes.c_int32),
        ("atoms", ctypes.c_int32),
        ("block", ctypes.c_int32),
        ("pbc_radius", ctypes.c_int32),
    ]


class MfGeometryArgs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "coords", "gram", "scale", "pad_mask", "pair_delta", "pair_dist2", "pair_dist", "pair_dist_norm",
        "mask_bits")] + [("cutoff", ctypes.c_float), ("batch", ctypes.c_int32), ("atoms", ctypes.c_int32),
                         ("pbc_radius", ctypes.c_int32), ("pair_mask", ctypes.c_void_p),
                         ("scale_mode", ctypes.c_int32)]


MF_SCALE_GIVEN = 0
MF_SCALE_RMS = 1
MF_LATTICE_Y1 = 0
MF_LATTICE_LTRI = 1


class MfRadiusAttnArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("mask_bits", ctypes.c_void_p),
        ("block_mask", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("out_f32", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("scale", ctypes.c_float),
        ("batch", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("atoms", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
    ]


class MfAdalnRowsArgs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("x", "y", "gate", "shift", "scale", "mol", "x_out", "h_out")] + [
        ("eps", ctypes.c_float)] + [(n, ctypes.c_int32) for n in ("tokens", "channels", "batch", "mod_stride", "dtype")]


class MfRowsToHeadsArgs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("rows", "slot", "heads")] + [("first_part_scale", ctypes.c_float)] + [
        (n, ctypes.c_int32) for n in ("tokens", "parts", "batch", "heads_count", "width", "head_dim", "src_dtype",
                                      "dst_dtype")]


class MfHeadsToRowsArgs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("heads", "row_index", "rows")] + [
        (n, ctypes.c_int32) for n in ("tokens", "batch", "heads_count", "width", "head_dim", "src_dtype", "dst_dtype")]


class MfPairMlpArgs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("pair_delta", "pair_dist_norm", "pair_mask", "rbf_centers")] + [
        ("rbf_gamma", ctypes.c_float)] + [(f"{m}_{t}", ctypes.c_void_p) for m in "uvw" for t in ("w1", "b1", "w2", "b2")] + [
        (n, ctypes.c_void_p) for n in ("u_out", "v_out", "w_out")] + [
        (n, ctypes.c_int32) for n in ("batch", "atoms", "rbf", "hidden", "heads")] + [
        ("n_freqs", ctypes.c_int32), ("freqs", ctypes.c_void_p), ("global_geom", ctypes.c_void_p)]


class MfPairMlpBwdArgs(ctypes.Structure):
    _fields_ = [("fwd", MfPairMlpArgs)] + [(f"{m}_grad", ctypes.c_void_p) for m in "uvw"] + [
        (f"{m}_{t}", ctypes.c_void_p) for m in "uvw" for t in ("dw1", "db1", "dw2", "db2")] + [
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_uint64)]


_LIB: ctypes.CDLL | None = None
_LOAD_ERROR: str | None = None


def _load() -> ctypes.CDLL | None:
    global _LIB, _LOAD_ERROR
    if _LIB is not None or _LOAD_ERROR is not None:
        return _LIB
    path = Path(os.environ.get("MF_HIP_LIBRARY", LIB_PATH))
    if not path.exists():
        _LOAD_ERROR = f"{path} is not built (run `python -m matterformer_amd.build`)"
        return None
    try:
        lib = ctypes.CDLL(str(path))
    except OSError as exc:
        _LOAD_ERROR = f"failed to load {path}: {exc}"
        return None
    lib.mf_abi_version.restype = ctypes.c_int
    lib.mf_last_error.restype = ctypes.c_char_p
    for name, argtype in (
        ("mf_simplicial_fwd", MfSimplicialFwdArgs),
        ("mf_simplicial_fwd_noalloc", MfSimplicialFwdArgs),
        ("mf_simplicial_bwd", MfSimplicialBwdArgs),
        ("mf_knn", MfKnnArgs),
        ("mf_knn_mask", MfKnnMaskArgs),
        ("mf_radius_mask", MfRadiusMaskArgs),
        ("mf_geometry_features", MfGeometryArgs),
        ("mf_radius_attn", MfRadiusAttnArgs),
        ("mf_adaln_rows", MfAdalnRowsArgs),
        ("mf_rows_to_heads", MfRowsToHeadsArgs),
        ("mf_heads_to_rows", MfHeadsToRowsArgs),
        ("mf_pair_mlp_bias", MfPairMlpArgs),
        ("mf_pair_mlp_bias_bwd", MfPairMlpBwdArgs),
    ):
        fn = getattr(lib, name, None)
        if fn is not None:
            fn.argtypes = [ctypes.POINTER(argtype), ctypes.c_void_p]
            fn.restype = ctypes.c_int
    lib.mf_simplicial_fwd_supported.argtypes = [ctypes.c_int32] * 5
    lib.mf_simplicial_fwd_supported.restype = ctypes.c_int
    lib.mf_simplicial_fwd_workspace_size.argtypes = [ctypes.c_int32] * 5
    lib.mf_simplicial_fwd_workspace_size.restype = ctypes.c_uint64
    lib.mf_simplicial_bwd_workspace_size.argtypes = [ctypes.c_int32] * 5
    lib.mf_simplicial_bwd_workspace_size.restype = ctypes.c_uint64
    if getattr(lib, "mf_pair_mlp_bias_bwd_workspace_size", None) is not None:
        lib.mf_pair_mlp_bias_bwd_workspace_size.argtypes = [ctypes.c_int32]
        lib.mf_pair_mlp_bias_bwd_workspace_size.restype = ctypes.c_uint64
    if getattr(lib, "mf_lattice_terms", None) is not None:
        lib.mf_lattice_terms.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32, ctypes.c_void_p,
                                         ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        lib.mf_lattice_terms.restype = ctypes.c_int
    version = lib.mf_abi_version()
    if version != EXPECTED_ABI_VERSION:
        _LOAD_ERROR = f"{path} has ABI version {version}, expected {EXPECTED_ABI_VERSION}"
        return None
    _LIB = lib
    return lib


def library_path() -> Path:
    return Path(os.environ.get("MF_HIP_LIBRARY", LIB_PATH))


def load_error() -> str | None:
    _load()
    return _LOAD_ERROR


def is_loaded() -> bool:
    return _load() is not None


def lib() -> ctypes.CDLL:
    handle = _load()
    if handle is None:
        raise RuntimeError(f"matterformer_amd HIP library unavailable: {_LOAD_ERROR}")
    return handle


def last_error() -> str:
    return lib().mf_last_error().decode("utf-8", errors="replace")


def check(status: int, what: str) -> None:
    if status != MF_OK:
        raise RuntimeError(f"{what} failed (status {status}): {last_error()}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dtype]
    except KeyError as exc:
        raise RuntimeError(f"unsupported dtype {dtype}; expected float16/bfloat16/float32") from exc


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def current_stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


_WORKSPACES: dict = {}
# Workspaces of calls recorded into HIP graphs.  A captured kernel keeps the
# address it was recorded with, so each captured call gets a buffer of its
# own that must outlive every replay: they are kept here until the process
# ends (a few hundred bytes per captured call on the pair-kernel path).
_CAPTURED_WORKSPACES: list = []


def workspace(nbytes: int, device: torch.device) -> torch.Tensor | None:
    """Device scratch for an entry point (16-byte aligned; torch's allocator
    hands out 512-byte aligned blocks).

    mf_simplicial_fwd's workspace holds a claim counter that must be zero
    before the first call and that every call leaves zero.  Eager calls keep
    one buffer per (device, stream) -- calls on one stream are ordered -- and
    zero-fill it whenever it is allocated or grown.

    A call made while the current stream is capturing a HIP graph gets a
    fresh buffer instead, zeroed by a fill kernel recorded into the same
    graph (so every replay starts from zero), which no eager call and no
    other captured call shares.  One graph replayed concurrently with itself
    on two streams would still share its own buffer; replays of one graph
    must be ordered."""
    if nbytes == 0:
        return None
    dev = torch.device(device)
    if torch.cuda.is_current_stream_capturing():
        buf = torch.zeros(int(nbytes), dtype=torch.uint8, device=dev)
        _CAPTURED_WORKSPACES.append(buf)
        return buf
    key = (dev.index if dev.index is not None else torch.cuda.current_device(),
           torch.cuda.current_stream(dev).cuda_stream)
    buf = _WORKSPACES.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.zeros(int(nbytes), dtype=torch.uint8, device=dev)
        _WORKSPACES[key] = buf
    return buf
