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
    return sorted(set(re.findall(r"^\s*(?:int|const char\*|uint64_t)\s+(mf_[a-z0-9_]+)\s*\(", text, flags=re.M)))


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


STRUCTS = {
    "mf_simplicial_fwd_args": _native.MfSimplicialFwdArgs,
    "mf_simplicial_bwd_args": _native.MfSimplicialBwdArgs,
    "mf_knn_args": _native.MfKnnArgs,
    "mf_knn_mask_args": _native.MfKnnMaskArgs,
    "mf_radius_mask_args": _native.MfRadiusMaskArgs,
    "mf_geometry_args": _native.MfGeometryArgs,
    "mf_radius_attn_args": _native.MfRadiusAttnArgs,
    "mf_adaln_rows_args": _native.MfAdalnRowsArgs,
    "mf_rows_to_heads_args": _native.MfRowsToHeadsArgs,
    "mf_heads_to_rows_args": _native.MfHeadsToRowsArgs,
    "mf_pair_mlp_args": _native.MfPairMlpArgs,
}


def test_ctypes_structs_match_the_header_layout(tmp_path):
    """Every argument struct of the ctypes binding has the C compiler's size and field offsets (gcc on the
    header itself), so a field added on one side only fails here, not as a wrong pointer on the GPU."""
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "mf_capi.h"', "int main(void) {"]
    for cname, py in STRUCTS.items():
        lines.append(f'  printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for fname, *_ in py._fields_:
            lines.append(f'  printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run([cc, f"-I{HEADER.parent}", str(src), "-o", str(exe)], check=True)
    got = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        cname, fname, val = line.split()
        got[(cname, fname)] = int(val)
    for cname, py in STRUCTS.items():
        assert got[(cname, "sizeof")] == ctypes.sizeof(py), cname
        for fname, *_ in py._fields_:
            assert got[(cname, fname)] == getattr(py, fname).offset, (cname, fname)


def test_backward_low_rank_arguments_are_validated_before_any_device_call():
    lib = _native.lib()
    fake = 1 << 20  # never dereferenced: every call below fails validation first
    a = _native.MfSimplicialBwdArgs(q=fake, k1=fake, v1=fake, k2=fake, v2=fake, grad_out=fake, out=fake, lse=fake,
                                    query_valid=fake, pair_key_valid=fake, batch=2, heads=2, tokens=8, head_dim=16,
                                    dtype=_native.MF_DTYPE_F32, grad_dtype=_native.MF_DTYPE_F32)
    a.dangle_left = fake
    assert lib.mf_simplicial_bwd(a, None) == _native.MF_ERR_INVALID_ARGUMENT
    assert "without an angle term" in _native.last_error()
    a.dangle_left = None
    a.angle_left, a.angle_right, a.angle_gate, a.angle_rank = fake, fake, fake, 65
    assert lib.mf_simplicial_bwd(a, None) == _native.MF_ERR_INVALID_ARGUMENT and "angle_rank" in _native.last_error()
    a.angle_left = None
    a.message_left, a.message_right, a.message_basis, a.message_rank = fake, fake, fake, 8
    need = lib.mf_simplicial_bwd_workspace_size(2, 2, 8, 16, 8)
    assert need == 2 * 2 * 2 * 8 * 8 * 4
    assert lib.mf_simplicial_bwd_workspace_size(2, 2, 8, 16, 0) == 0
    a.workspace, a.workspace_bytes = fake, need - 4
    assert lib.mf_simplicial_bwd(a, None) == _native.MF_ERR_INVALID_ARGUMENT and "workspace" in _native.last_error()
