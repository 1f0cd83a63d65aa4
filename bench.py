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
  roofline      the entry point's achieved TFLOP/s against the bf16 dense MFMA
                peak: valid FLOPs over the average duration of one
                mf_simplicial_fwd launch (the pair kernel), timed with HIP
                events on the launch stream; `traffic` is the HBM bytes of
                one such launch from the committed rocprofv3 --pmc summary
                (profiles/simplicial_fwd_geom_traffic.json) when present;
  cpu_baseline  the oracle's torch-CPU restatement of the reference path
                (padded N, chunk 128, bf16 as configured) on the whole batch.

Other workloads (one JSON line each, not the headline):
  --workload knn          kNN top-16 at B=32 and scaled to
                          B=32*1024 for the HBM roofline;
  --workload radius       radius mask + radius attention;
  --copy-calibration      a plain device copy of known size, run under
                          rocprofv3 --pmc to scale FETCH_SIZE / WRITE_SIZE.
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
    ap.add_argument("--cpu-sample", type=int, default=64, help="molecules in the CPU-baseline sample (0 = skip)")
    ap.add_argument("--cpu-threads", type=int, default=0, help="CPU-baseline threads (0 = min(16, cores))")
    ap.add_argument("--workload", choices=("simplicial", "knn", "radius"), default="simplicial")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run a plain 512 MiB device copy (for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
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
    passes = 0
    t0 = time.perf_counter()
    # whole passes over the sample until about 10 s of CPU work (at most 5)
    while passes < 5 and (passes == 0 or time.perf_counter() - t0 < 10.0):
        for s in range(0, sample, group):
            e = min(sample, s + group)
            reference_path(*(t[s:e] for t in bf), workload.query_valid[s:e], workload.pair_key_valid[s:e],
                           chunk_size=128)
        passes += 1
    elapsed = time.perf_counter() - t0
    n = workload.counts[:sample].to(torch.int64)
    flops = passes * 4 * workload.q.shape[1] * workload.q.shape[3] * int((n ** 3).sum())
    return {
        "value": flops / elapsed / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{passes} pass(es) over the first {sample} of the 64 GEOM molecules, bf16, padded N=181, "
                   f"chunk_size 128, torch CPU restatement of simplicial_attention_torch_from_projected; "
                   f"{elapsed:.2f} s"),
        "molecules_per_s": passes * sample / elapsed,
        "seconds": elapsed,
    }


def event_times(stream, fn, launches: int):
    """Median and mean duration (ms) of single launches of fn, one HIP event pair
    each, recorded on the stream the kernels run on."""
    import torch

    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(launches)]
    for a, b in evs:
        a.record(stream)
        fn()
        b.record(stream)
    torch.cuda.synchronize()
    t = sorted(a.elapsed_time(b) for a, b in evs)
    return t[len(t) // 2], sum(t) / len(t)


def graph_times(stream, fn, per_graph: int = 20, replays: int = 10):
    """Mean duration (ms) of one call of fn when calls run back to back: fn is
    captured per_graph times into one HIP graph, and one event pair on the
    launch stream brackets `replays` replays.  For kernels of a few
    microseconds a per-launch event pair mostly measures the host's launch
    latency; this figure is the device time of the kernels."""
    import torch

    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(per_graph):
            fn()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        g.replay()
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(replays):
            g.replay()
        stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / (replays * per_graph)


def timed_loop(stream, fn, steps: int, warmup: int):
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        fn()
    stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps, time.perf_counter() - t0


def copy_calibration() -> int:
    """512 MiB device-to-device copy, 5 launches: FETCH_SIZE and WRITE_SIZE of
    one dispatch should each read 524288 KiB on an exact counter."""
    import torch

    dev = torch.device("cuda", 0)
    n = 512 * 1024 * 1024 // 4
    src = torch.arange(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    assert torch.equal(dst[-4:], src[-4:])
    print(json.dumps({"copy_bytes": n * 4, "launches": 5}), flush=True)
    return 0


def bench_knn(args) -> int:
    import torch

    from matterformer_amd.geometry_ops import knn_graph
    from matterformer_amd.workloads import knn_workload

    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    small = knn_workload()
    scaled = knn_workload(batch=32 * 1024)
    res = {}
    for name, w in (("c3", small), ("scaled", scaled)):
        c = w.coords.to(dev)
        B, N, _ = c.shape
        step = lambda: knn_graph(c, w.k)  # noqa: E731
        ms, _ = timed_loop(stream, step, args.steps, args.warmup)
        med, _ = event_times(stream, step, 50)
        nbytes = B * N * 3 * 4 + B * N * w.k * 8
        res[name] = {"B": B, "ms": ms, "kernel_ms": med, "bytes": nbytes, "queries": B * N}
    cpu = None
    if args.cpu_sample > 0:
        from oracle.native import knn as oracle_knn

        n_cpu = min(args.cpu_sample * 128, scaled.coords.shape[0])
        sample = scaled.coords[:n_cpu].numpy()
        t0 = time.perf_counter()
        oracle_knn(sample, scaled.k)
        el = time.perf_counter() - t0
        cpu = {"value": n_cpu * 181 / el, "unit": "queries/s", "cores": 1, "kind": "port",
               "sample": f"oracle/knn.c (gcc -O2, 1 thread) on {n_cpu} molecules x 181 atoms, k=16; {el:.2f} s"}
    sc = res["scaled"]
    achieved = sc["bytes"] / (sc["kernel_ms"] * 1e-3) / 1e9
    line = {
        "metric": "kNN top-16 queries/s (configs[2] scaled to 32768 molecules)",
        "value": round(sc["queries"] / (sc["ms"] * 1e-3), 1),
        "unit": "queries/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(sc["ms"], 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seeded, BASELINE.json configs[2])",
        "config": {"workload": "kNN top-16, 181 atoms/molecule, coords N(0, 2 A^2)", "batch": sc["B"], "atoms": 181,
                   "k": 16, "c3_batch32_ms": round(res["c3"]["ms"], 5)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": committed_traffic("knn_c3_scaled"),
                     "kernel": "mf::knn::knn_block_kernel<16, 1>", "kernel_ms": round(sc["kernel_ms"], 5)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def bench_radius(args) -> int:
    import torch

    from matterformer_amd.geometry_ops import lattice_to_gram, radius_attention, radius_mask
    from matterformer_amd.workloads import radius_workload

    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev)
    w = radius_workload()
    frac = w.frac.to(dev)
    gram = lattice_to_gram(w.lattice.to(dev))
    q, k, v = (t.to(torch.bfloat16).to(dev) for t in (w.q, w.k, w.v))
    bits, blocks = radius_mask(frac, w.cutoff, gram=gram)
    pairs = 0
    words = bits.cpu().numpy().view("uint32")
    import numpy as np

    pairs = int(np.unpackbits(words.view(np.uint8)).sum())
    B, H, N, D = q.shape
    mask_step = lambda: radius_mask(frac, w.cutoff, gram=gram)  # noqa: E731
    attn_step = lambda: radius_attention(q, k, v, bits, blocks)  # noqa: E731
    both = lambda: radius_attention(q, k, v, *radius_mask(frac, w.cutoff, gram=gram))  # noqa: E731
    ms, _ = timed_loop(stream, both, args.steps, args.warmup)
    mask_launch_ms, _ = event_times(stream, mask_step, 50)
    attn_launch_ms, _ = event_times(stream, attn_step, 50)
    mask_ms = graph_times(stream, mask_step)
    attn_ms = graph_times(stream, attn_step)
    graph_step_ms = graph_times(stream, both)
    flops = w.attention_flops(pairs)
    attn_bytes = 4 * B * H * N * D * 2 + bits.numel() * 4 + blocks.numel()
    achieved = attn_bytes / (attn_ms * 1e-3) / 1e9
    cpu = None
    if args.cpu_sample > 0:
        from oracle.native import radius_mask as oracle_radius_mask
        from oracle.native import unpack_bits
        from oracle.radius import masked_attention_fp64

        g = gram.cpu().numpy()
        t0 = time.perf_counter()
        rb, _ = oracle_radius_mask(w.frac.numpy(), w.cutoff, gram=g)
        masked_attention_fp64(*(t.float().cpu().numpy() for t in (q, k, v)), unpack_bits(rb, N), D ** -0.5)
        el = time.perf_counter() - t0
        cpu = {"value": B / el, "unit": "cells/s", "cores": 1, "kind": "port",
               "sample": f"oracle radius mask (C, 1 thread) + float64 numpy masked softmax, all 8 cells; {el:.2f} s"}
    line = {
        "metric": "radius mask + radius attention cells/s (configs[3])",
        "value": round(B / (ms * 1e-3), 1), "unit": "cells/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded, BASELINE.json configs[3])",
        "config": {"workload": "periodic MOF cells, 6 A cutoff, minimum image, 64-atom tiles", "cells": B,
                   "atoms": N, "heads": H, "head_dim": D, "allowed_pairs": pairs,
                   "mask_ms": round(mask_ms, 5), "attn_ms": round(attn_ms, 5),
                   "mask_single_launch_ms": round(mask_launch_ms, 5),
                   "attn_single_launch_ms": round(attn_launch_ms, 5),
                   "graph_replay_ms_per_step": round(graph_step_ms, 5),
                   "attn_valid_gflop": round(flops / 1e9, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": committed_traffic("radius_attn_c4"),
                     "kernel": "mf::rattn::radius_attn_pair_kernel<bf16, 64, true>", "kernel_ms": round(attn_ms, 5)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def main() -> int:
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}); "
              "every kernel here works per molecule or per cell with no cross-GPU exchange, "
              "see DESIGN.md for how the path would shard.", file=sys.stderr)
        return 2

    import torch

    from matterformer_amd import _native
    from matterformer_amd.workloads import simplicial_workload

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    if args.copy_calibration:
        return copy_calibration()
    if args.workload == "knn":
        return bench_knn(args)
    if args.workload == "radius":
        return bench_radius(args)
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

    ms_per_step, wall = timed_loop(stream, step, args.steps, args.warmup)

    flops = w.valid_flops()
    tflops = flops / (ms_per_step * 1e-3) / 1e12
    atoms = int(w.counts.sum())

    # Per-launch duration of the launch sequence: one event pair per launch on
    # the launch stream (median and mean of 100 launches).
    kernel_ms, kernel_mean_ms = event_times(stream, step, 100)
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
            "kernel": "mf_simplicial_fwd launch: simplicial_pair_kernel<bf16, 64, pair_valid=0>",
            "kernel_ms": round(kernel_ms, 5),
            "kernel_mean_ms": round(kernel_mean_ms, 5),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
