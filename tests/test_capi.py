"""C-ABI surface of libmf_hip.so: loads, exports every declared symbol, validates arguments.

CPU only: nothing here launches a kernel.
"""

import ctypes
import re
from pathlib import Path

import pytest

from matterformer_amd import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "mf_capi.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(mf_[a-z0-9_]+)\s*\(", text, flags=re.M)))


def test_library_is_built_and_loads():
    assert _native.library_path().exists(), "run python -m matterformer_amd.build"
    assert _native.is_loaded(), _native.load_error()


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert "mf_simplicial_fwd" in names and "mf_last_error" in names
    lib = ctypes.CDLL(str(_native.library_path()))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared in mf_capi.h but not exported: {missing}"


def test_abi_version_matches_header():
    m = re.search(r"#define\s+MF_ABI_VERSION\s+(\d+)", HEADER.read_text())
    assert m is not None
    assert _native.lib().mf_abi_version() == int(m.group(1)) == _native.EXPECTED_ABI_VERSION


def test_null_args_rejected_with_message():
    lib = _native.lib()
    status = lib.mf_simplicial_fwd(None, None)
    assert status == _native.MF_ERR_INVALID_ARGUMENT
    assert "args is NULL" in _native.last_error()


def test_missing_operands_rejected_before_any_device_call():
    args = _native.MfSimplicialFwdArgs()
    args.batch, args.heads, args.tokens, args.head_dim = 1, 1, 4, 8
    status = _native.lib().mf_simplicial_fwd(args, None)
    assert status == _native.MF_ERR_INVALID_ARGUMENT
    assert "must be non-NULL" in _native.last_error()


def test_check_raises_runtime_error_with_library_message():
    _native.lib().mf_simplicial_fwd(None, None)
    with pytest.raises(RuntimeError, match="args is NULL"):
        _native.check(_native.MF_ERR_INVALID_ARGUMENT, "mf_simplicial_fwd")


@pytest.mark.parametrize("name,argtype", [("mf_knn", _native.MfKnnArgs), ("mf_radius_mask", _native.MfRadiusMaskArgs),
                                          ("mf_radius_attn", _native.MfRadiusAttnArgs)])
def test_geometry_entry_points_reject_null_and_missing_pointers(name, argtype):
    fn = getattr(_native.lib(), name)
    assert fn(None, None) == _native.MF_ERR_INVALID_ARGUMENT
    assert "args is NULL" in _native.last_error()
    assert fn(argtype(), None) == _native.MF_ERR_INVALID_ARGUMENT
    assert "must be non-NULL" in _native.last_error()


def test_geometry_entry_points_validate_sizes_before_any_device_call():
    lib = _native.lib()
    fake = 1 << 20  # never dereferenced: every call below fails validation first
    a = _native.MfKnnArgs(coords=fake, idx=fake, batch=1, atoms=4, k=65)
    assert lib.mf_knn(a, None) == _native.MF_ERR_INVALID_ARGUMENT and "k must be in [1, 64]" in _native.last_error()
    r = _native.MfRadiusMaskArgs(coords=fake, mask_bits=fake, batch=1, atoms=4, block=48, cutoff=1.0, pbc_radius=1)
    assert lib.mf_radius_mask(r, None) == _native.MF_ERR_INVALID_ARGUMENT and "block" in _native.last_error()
    r.block, r.cutoff = 64, -1.0
    assert lib.mf_radius_mask(r, None) == _native.MF_ERR_INVALID_ARGUMENT and "cutoff" in _native.last_error()
    r.cutoff, r.gram, r.pbc_radius = 1.0, fake, 3
    assert lib.mf_radius_mask(r, None) == _native.MF_ERR_INVALID_ARGUMENT and "pbc_radius" in _native.last_error()
    t = _native.MfRadiusAttnArgs(q=fake, k=fake, v=fake, mask_bits=fake, out=fake, scale=0.125, batch=1, heads=1,
                                 atoms=4, head_dim=64, dtype=_native.MF_DTYPE_F32)
    assert lib.mf_radius_attn(t, None) == _native.MF_ERR_UNSUPPORTED
    assert "float16/bfloat16" in _native.last_error()
    t.dtype, t.head_dim = _native.MF_DTYPE_BF16, 48
    assert lib.mf_radius_attn(t, None) == _native.MF_ERR_UNSUPPORTED and "head_dim" in _native.last_error()
