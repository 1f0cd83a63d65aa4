"""mf_simplicial_fwd_noalloc (the allocation-free entry point) against mf_simplicial_fwd, through the C ABI.

The variant runs the same kernels with the scratch in a static per-GPU device
array instead of a caller workspace, so its outputs must equal the
workspace entry point's bit for bit.  Two calls in a row, the second on a
smaller input (the array keeps the first call's contents), on each 16-bit
path (pair kernel, N > 512 kernel) and on the fp32 path, plus the size limit.
"""

import ctypes

import pytest
import torch

from matterformer_amd import _native
from matterformer_amd.workloads import random_simplicial, simplicial_workload

pytestmark = pytest.mark.gpu


def _inputs(case, dtype, device):
    q, k1, v1, k2, v2, qv, pkv, pv = case
    ops = [t.to(dtype).to(device).contiguous() for t in (q, k1, v1, k2, v2)]
    masks = [qv.to(torch.uint8).to(device), pkv.to(torch.uint8).to(device),
             None if pv is None else pv.to(torch.uint8).to(device)]
    return ops, masks


def _call(entry, ops, masks, dtype, precision, workspace=None):
    B, H, N, D = ops[0].shape
    dev = ops[0].device
    out = torch.full((B, H, N, D), float("nan"), dtype=dtype, device=dev)
    out32 = torch.full((B, H, N, D), float("nan"), dtype=torch.float32, device=dev)
    lse = torch.full((B, H, N), float("nan"), dtype=torch.float32, device=dev)
    args = _native.MfSimplicialFwdArgs(
        q=ops[0].data_ptr(), k1=ops[1].data_ptr(), v1=ops[2].data_ptr(), k2=ops[3].data_ptr(), v2=ops[4].data_ptr(),
        query_valid=masks[0].data_ptr(), pair_key_valid=masks[1].data_ptr(),
        pair_valid=None if masks[2] is None else masks[2].data_ptr(),
        out=out.data_ptr(), out_f32=out32.data_ptr(), lse=lse.data_ptr(),
        workspace=None if workspace is None else workspace.data_ptr(),
        workspace_bytes=0 if workspace is None else workspace.numel(),
        batch=B, heads=H, tokens=N, head_dim=D, dtype=_native.dtype_code(dtype),
        precision=_native.MF_PREC[precision])
    status = getattr(_native.lib(), entry)(ctypes.byref(args), _native.current_stream(dev))
    _native.check(status, entry)
    torch.cuda.synchronize()
    return out, out32, lse


def _reference(ops, masks, dtype, precision):
    B, H, N, D = ops[0].shape
    nbytes = _native.lib().mf_simplicial_fwd_workspace_size(B, H, N, D, _native.dtype_code(dtype))
    ws = torch.zeros(max(int(nbytes), 16), dtype=torch.uint8, device=ops[0].device)
    return _call("mf_simplicial_fwd", ops, masks, dtype, precision, ws)


def _check_pair(cuda, first, second, dtype, precision):
    for name, case in (("first", first), ("second", second)):
        print(f"noalloc {name}: shape {tuple(case[0].shape)} {dtype} {precision}", flush=True)
        ops, masks = _inputs(case, dtype, cuda)
        got = _call("mf_simplicial_fwd_noalloc", ops, masks, dtype, precision)
        ref = _reference(ops, masks, dtype, precision)
        for g, r in zip(got, ref):
            assert torch.equal(g, r), name


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
def test_noalloc_pair_kernel_path(cuda, dtype):
    w = simplicial_workload("geom", batch=24)
    first = (w.q, w.k1, w.v1, w.k2, w.v2, w.query_valid, w.pair_key_valid, None)
    second = random_simplicial(3, 2, 40, 64, seed=5, counts=[40, 17, 3], holes=[(0, 2)], std=0.2)
    _check_pair(cuda, first, second, dtype, "bf16_tc")


def test_noalloc_long_molecule_path(cuda):
    first = random_simplicial(2, 2, 600, 64, seed=6, counts=[600, 540], pair_drop=0.1, std=0.05)
    second = random_simplicial(1, 2, 520, 32, seed=7, counts=[513], std=0.05)
    _check_pair(cuda, first, second, torch.bfloat16, "bf16_tc")


def test_noalloc_fp32_path(cuda):
    first = random_simplicial(4, 2, 29, 32, seed=8, counts=[29, 20, 9, 1], std=0.5)
    second = random_simplicial(2, 1, 9, 16, seed=9, counts=[9, 4], std=0.5)
    _check_pair(cuda, first, second, torch.float32, "ieee_fp32")


def test_noalloc_rejects_shapes_beyond_its_scratch(cuda):
    # 1024 molecules of 600 tokens need ~44 MB of scratch on the N > 512 path: refused on the host
    B, H, N, D = 1024, 8, 600, 64
    need = _native.lib().mf_simplicial_fwd_workspace_size(B, H, N, D, _native.MF_DTYPE_BF16)
    assert need > (8 << 20)
    args = _native.MfSimplicialFwdArgs(batch=B, heads=H, tokens=N, head_dim=D, dtype=_native.MF_DTYPE_BF16,
                                       precision=0)
    status = _native.lib().mf_simplicial_fwd_noalloc(ctypes.byref(args), _native.current_stream(cuda))
    assert status == _native.MF_ERR_UNSUPPORTED
    assert "static scratch" in _native.last_error()
