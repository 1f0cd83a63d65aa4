#!/usr/bin/env python
"""Benchmark of the 2-simplicial attention forward on one MI355X.

Workload ("C2"): GEOM-Drugs-like batch of 64
molecules, atom counts round(44 + 12 z) clipped to [10, 181], padded to N=181,
8 heads, head_dim 64, bf16 inputs randn/8, seed 1; softmax over all valid
(j,k) pairs.  A step is one forward launch of mf_simplicial_fwd over the batch
(inference mode: the bf16 output, no saved fp32 output / lse), with inputs
already resident in HBM.

value = valid FLOPs (sum_b 4 H D n_b^3) / step time, in TFLOP/s.

Prints ONE JSON line.  Also reports:
  roofline      the kernel's achieved TFLOP/s against the bf16 dense MFMA peak,
                timed with HIP events on the launch stream; `traffic` comes from
                the committed rocprofv3 --pmc summary when present;
  cpu_baseline  the oracle's torch-CPU restatement of the reference path
                (padded N, chunk 128, bf16 as configured) on a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

BF16_DENSE_PEAK_TFLOPS = 2516.6
HBM_PEAK_GBS = 8000.0
PROFILES = ROOT / "profiles"


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-sample", type=int, default=32, help="molecules in the CPU-baseline sample (0 = skip)")
    ap.add_argument("--cpu-threads", type=int, default=0, help="CPU-baseline threads (0 = min(16, cores))")
    return ap.parse_args()


def committed_traffic(name: str):
    """HBM bytes per launch from profiles/<name>_traffic.json (rocprofv3 --pmc), or None."""
    path = PROFILES / f"{name}_traffic.json"
    if not path.exists():
        return None
    try:
        return json.loads(path.read_text()).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def cpu_baseline(workload, sample: int, threads: int):
    import torch

    from oracle.simplicial import reference_path

    sample = min(sample, workload.q.shape[0])
    threads = threads or min(16, os.cpu_count() or 1)
    torch.set_num_threads(threads)
    bf = [t[:sample].to(torch.bfloat16) for t in (workload.q, workload.k1, workload.v1, workload.k2, workload.v2)]
    group = 8
    t0 = time.perf_counter()
    for s in range(0, sample, group):
        e = min(sample, s + group)
        reference_path(*(t[s:e] for t in bf), workload.query_valid[s:e], workload.pair_key_valid[s:e],
                       chunk_size=128)
    elapsed = time.perf_counter() - t0
    n = workload.counts[:sample].to(torch.int64)
    flops = 4 * workload.q.shape[1] * workload.q.shape[3] * int((n ** 3).sum())
    return {
        "value": flops / elapsed / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"first {sample} of the 64 GEOM molecules, bf16, padded N=181, chunk_size 128, "
                   f"torch CPU restatement of simplicial_attention_torch_from_projected; {elapsed:.2f} s"),
        "molecules_per_s": sample / elapsed,
        "seconds": elapsed,
    }


def main() -> int:
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}); "
              "the simplicial forward has no cross-GPU exchange, see DESIGN.md for how it shards.",
              file=sys.stderr)
        return 2

    import torch

    from matterformer_amd import _native
    from matterformer_amd.workloads import simplicial_workload

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    lib = _native.lib()

    w = simplicial_workload("geom")
    wd = w.to(dev, torch.bfloat16)
    B, H, N, D = wd.shape
    ops = [t.contiguous() for t in (wd.q, wd.k1, wd.v1, wd.k2, wd.v2)]
    out = torch.empty((B, H, N, D), device=dev, dtype=torch.bfloat16)
    ws_bytes = lib.mf_simplicial_fwd_workspace_size(B, H, N, D, _native.MF_DTYPE_BF16)
    ws = _native.workspace(ws_bytes, dev)
    args_struct = _native.MfSimplicialFwdArgs(
        q=ops[0].data_ptr(), k1=ops[1].data_ptr(), v1=ops[2].data_ptr(), k2=ops[3].data_ptr(), v2=ops[4].data_ptr(),
        query_valid=wd.query_valid.data_ptr(), pair_key_valid=wd.pair_key_valid.data_ptr(), pair_valid=None,
        out=out.data_ptr(), out_f32=None, lse=None,
        workspace=None if ws is None else ws.data_ptr(), workspace_bytes=ws_bytes,
        batch=B, heads=H, tokens=N, head_dim=D,
        dtype=_native.MF_DTYPE_BF16, precision=_native.MF_PREC["bf16_tc"],
    )
    stream = torch.cuda.current_stream(dev)
    handle = stream.cuda_stream
    fwd = lib.mf_simplicial_fwd

    def step():
        st = fwd(args_struct, handle)
        if st != 0:
            raise RuntimeError(f"mf_simplicial_fwd failed: {_native.last_error()}")

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(args.steps):
        step()
    stop.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = start.elapsed_time(stop)
    ms_per_step = gpu_ms / args.steps

    flops = w.valid_flops()
    tflops = flops / (ms_per_step * 1e-3) / 1e12
    atoms = int(w.counts.sum())

    # Per-launch kernel time: one event pair per launch, averaged (same stream).
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(50)]
    for a, b in evs:
        a.record(stream)
        step()
        b.record(stream)
    torch.cuda.synchronize()
    kernel_ms = sorted(a.elapsed_time(b) for a, b in evs)[len(evs) // 2]
    achieved = flops / (kernel_ms * 1e-3) / 1e12

    cpu = cpu_baseline(w, args.cpu_sample, args.cpu_threads) if args.cpu_sample > 0 else None

    line = {
        "metric": "2-simplicial attn fwd TFLOP/s (%MFMA peak) + molecules/s, GEOM-Drugs shape",
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded, BASELINE.json configs[1])",
        "config": {
            "workload": "GEOM-Drugs-like 2-simplicial attention fwd (configs[1])",
            "batch": B, "heads": H, "tokens_padded": N, "head_dim": D,
            "valid_atoms": atoms, "valid_gflop": round(flops / 1e9, 4),
        },
        "pct_mfma_peak": round(100.0 * tflops / BF16_DENSE_PEAK_TFLOPS, 3),
        "molecules_per_s": round(B / (ms_per_step * 1e-3), 1),
        "atoms_per_s": round(atoms / (ms_per_step * 1e-3), 1),
        "wall_s": round(wall, 4),
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": BF16_DENSE_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / BF16_DENSE_PEAK_TFLOPS, 5),
            "traffic": committed_traffic("simplicial_fwd_geom"),
            "kernel": "mf::simplicial::simplicial_fwd_kernel<__bf16, 64>",
            "kernel_ms": round(kernel_ms, 5),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
