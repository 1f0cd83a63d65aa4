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
  roofline      the pair kernel's achieved TFLOP/s against the bf16 dense MFMA
                peak: valid FLOPs over the kernel's duration, taken from HIP
                events on the launch stream around replays of a graph of 20
                back-to-back launches (so launch latency is not counted);
                `traffic` is the HBM bytes of one launch from the committed
                rocprofv3 --pmc summary (profiles/simplicial_fwd_geom_traffic.json);
  cpu_baseline  the oracle's torch-CPU restatement of the reference path
                (padded N, chunk 128, bf16 as configured) on the host's physical
                cores (bounded by the box's share), plus a single-thread figure,
                the CPU model and the peak RSS;
  extra         the other configurations and calls, each timed the same way
                (graph replays) with its own roofline where one applies:
                the training-state forward (fp32 out + lse), forward + backward
                (mf_simplicial_bwd), C2 with a factorized bias, C1 (fp32),
                C3 kNN (and its HBM-sized scaled batch), C4 radius mask +
                attention, the configs[4] trunk forward (molecules/s), and the
                SimplicialAttention module on C2's batch (in_proj -> attention
                -> out_proj, eager, forward and train step).

Other entry modes (one JSON line each, not the headline):
  --workload knn          kNN top-16 at B=32 and scaled to
                          B=32*1024 for the HBM roofline;
  --workload radius       radius mask + radius attention;
  --workload trunk        the configs[4] trunk forward;
  --workload module       the TwoSimplicialAttention module (in_proj -> attention ->
                          out_proj) over the reference harness's grid
                          (scripts/benchmark_simplicial_attention.py:27-42), forward
                          and train step, modes none / factorized, impl hip and torch;
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
FP32_MFMA_PEAK_TFLOPS = 157.3
HBM_PEAK_GBS = 8000.0
PROFILES = ROOT / "profiles"


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # ~70 ms of untimed steps: the GPU reaches its steady-state clocks only after some tens of milliseconds
    # of work (20 warm-up steps measured 33.7-34.1 us per step, 2000 measured 30.8-30.9 us, same build)
    ap.add_argument("--warmup", type=int, default=2000)
    ap.add_argument("--cpu-sample", type=int, default=64, help="molecules in the CPU-baseline sample (0 = skip)")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="CPU-baseline threads (0 = physical cores, capped by OMP_NUM_THREADS when set)")
    ap.add_argument("--workload", choices=("simplicial", "knn", "radius", "trunk", "module"), default="simplicial")
    ap.add_argument("--no-extra", action="store_true", help="headline only (skip the extra configurations)")
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


def host_cpu() -> dict:
    """Physical cores (distinct (socket, core) pairs of lscpu -p) and the CPU model."""
    import subprocess

    info = {"physical_cores": os.cpu_count() or 1, "model": "unknown"}
    try:
        out = subprocess.run(["lscpu", "-p=SOCKET,CORE"], capture_output=True, text=True, timeout=10).stdout
        cores = {line for line in out.splitlines() if line and not line.startswith("#")}
        if cores:
            info["physical_cores"] = len(cores)
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                info["model"] = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return info


def _cpu_passes(workload, sample: int, seconds: float, max_passes: int = 5):
    import torch

    from oracle.simplicial import reference_path

    bf = [t[:sample].to(torch.bfloat16) for t in (workload.q, workload.k1, workload.v1, workload.k2, workload.v2)]
    group = 8
    passes = 0
    t0 = time.perf_counter()
    while passes < max_passes and (passes == 0 or time.perf_counter() - t0 < seconds):
        for s in range(0, sample, group):
            e = min(sample, s + group)
            reference_path(*(t[s:e] for t in bf), workload.query_valid[s:e], workload.pair_key_valid[s:e],
                           chunk_size=128)
        passes += 1
    return passes, time.perf_counter() - t0


def cpu_baseline(workload, sample: int, threads: int):
    import resource

    import torch

    host = host_cpu()
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = threads or (min(host["physical_cores"], share) if share > 0 else host["physical_cores"])
    sample = min(sample, workload.q.shape[0])
    n = workload.counts.to(torch.int64)
    H, D = workload.q.shape[1], workload.q.shape[3]
    torch.set_num_threads(threads)
    passes, elapsed = _cpu_passes(workload, sample, 10.0)
    flops = passes * 4 * H * D * int((n[:sample] ** 3).sum())
    # single thread on the first 8 molecules
    torch.set_num_threads(1)
    single_sample = min(8, sample)
    p1, e1 = _cpu_passes(workload, single_sample, 5.0, max_passes=3)
    f1 = p1 * 4 * H * D * int((n[:single_sample] ** 3).sum())
    torch.set_num_threads(threads)
    rss_gb = resource.getrusage(resource.RUSAGE_SELF).ru_maxrss / 1e6
    return {
        "value": flops / elapsed / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{passes} pass(es) over the first {sample} of the 64 GEOM molecules, bf16, padded N=181, "
                   f"chunk_size 128, torch CPU restatement of simplicial_attention_torch_from_projected, "
                   f"{threads} threads; {elapsed:.2f} s"),
        "molecules_per_s": passes * sample / elapsed,
        "seconds": elapsed,
        "cpu_model": host["model"],
        "physical_cores": host["physical_cores"],
        "single_thread": {"value": f1 / e1 / 1e12, "unit": "TFLOP/s", "molecules_per_s": p1 * single_sample / e1,
                          "sample": f"{p1} pass(es) over the first {single_sample} molecules; {e1:.2f} s"},
        "peak_rss_gb": round(rss_gb, 3),
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


def _graph_ms(fn, per_graph: int = 20, replays: int = 10) -> float:
    import torch

    return graph_times(torch.cuda.current_stream(), fn, per_graph=per_graph, replays=replays)


def measure_knn(cpu_sample: int) -> dict:
    """C3 (B=32) and the HBM-sized scaled batch (B=32*1024): graph-replayed times and the HBM roofline."""
    import torch

    from matterformer_amd.geometry_ops import knn_graph
    from matterformer_amd.workloads import knn_workload

    dev = torch.device("cuda", 0)
    res = {}
    for name, w, per_graph in (("c3", knn_workload(), 20), ("scaled", knn_workload(batch=32 * 1024), 2)):
        c = w.coords.to(dev)
        B, N, _ = c.shape
        ms = _graph_ms(lambda: knn_graph(c, w.k), per_graph=per_graph, replays=5)  # noqa: B023
        nbytes = B * N * 3 * 4 + B * N * w.k * 8
        res[name] = {"batch": B, "ms": ms, "bytes": nbytes, "queries": B * N}
    sc = res["scaled"]
    achieved = sc["bytes"] / (sc["ms"] * 1e-3) / 1e9
    cpu = None
    if cpu_sample > 0:
        from oracle.native import knn as oracle_knn

        w = knn_workload(batch=32 * 1024)
        n_cpu = min(cpu_sample * 128, w.coords.shape[0])
        t0 = time.perf_counter()
        oracle_knn(w.coords[:n_cpu].numpy(), w.k)
        el = time.perf_counter() - t0
        cpu = {"value": n_cpu * 181 / el, "unit": "queries/s", "cores": 1, "kind": "port",
               "sample": f"oracle/knn.c (gcc -O2, 1 thread) on {n_cpu} molecules x 181 atoms, k=16; {el:.2f} s"}
    return {
        "c3_ms": round(res["c3"]["ms"], 5), "scaled_batch": sc["batch"], "scaled_ms": round(sc["ms"], 5),
        "queries_per_s": round(sc["queries"] / (sc["ms"] * 1e-3), 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": committed_traffic("knn_c3_scaled"),
                     "kernel": "mf::knn::knn_code_kernel<16, 1>", "kernel_ms": round(sc["ms"], 5),
                     "algorithmic_bytes": sc["bytes"]},
        "cpu_baseline": cpu,
    }


def measure_radius(cpu_sample: int) -> dict:
    import numpy as np
    import torch

    from matterformer_amd.geometry_ops import lattice_to_gram, radius_attention, radius_mask
    from matterformer_amd.workloads import radius_workload

    dev = torch.device("cuda", 0)
    w = radius_workload()
    frac = w.frac.to(dev)
    gram = lattice_to_gram(w.lattice.to(dev))
    q, k, v = (t.to(torch.bfloat16).to(dev) for t in (w.q, w.k, w.v))
    bits, blocks = radius_mask(frac, w.cutoff, gram=gram)
    pairs = int(np.unpackbits(bits.cpu().numpy().view(np.uint32).view(np.uint8)).sum())
    B, H, N, D = q.shape
    mask_ms = _graph_ms(lambda: radius_mask(frac, w.cutoff, gram=gram))
    attn_ms = _graph_ms(lambda: radius_attention(q, k, v, bits, blocks))
    step_ms = _graph_ms(lambda: radius_attention(q, k, v, *radius_mask(frac, w.cutoff, gram=gram)))
    attn_bytes = 4 * B * H * N * D * 2 + bits.numel() * 4 + blocks.numel()
    achieved = attn_bytes / (attn_ms * 1e-3) / 1e9
    cpu = None
    if cpu_sample > 0:
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
    return {
        "cells": B, "atoms": N, "allowed_pairs": pairs, "mask_ms": round(mask_ms, 5), "attn_ms": round(attn_ms, 5),
        "step_ms": round(step_ms, 5), "cells_per_s": round(B / (step_ms * 1e-3), 1),
        "attn_valid_gflop": round(w.attention_flops(pairs) / 1e9, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 5), "traffic": committed_traffic("radius_attn_c4"),
                     "kernel": "mf::rattn::radius_attn_pair_kernel<bf16, 64, POS=true, QW=2>", "kernel_ms": round(attn_ms, 5),
                     "algorithmic_bytes": attn_bytes},
        "cpu_baseline": cpu,
    }


def measure_geometry() -> dict:
    """The one-pass geometry features (mf_geometry_features behind the mirrored adapters): configs[3]'s
    periodic cells (27 images, with the 6 A cutoff bits) and configs[1]'s GEOM molecules (non-periodic),
    graph-replayed, against the HBM roofline of the pair tensors they write (delta, d2, d, d_norm in fp32,
    plus the bits)."""
    import torch

    from matterformer_amd.geometry import NonPeriodicGeometryAdapter, PeriodicGeometryAdapter
    from matterformer_amd.workloads import radius_workload, simplicial_workload

    dev = torch.device("cuda", 0)
    rw = radius_workload()
    frac, lat = rw.frac.to(dev), rw.lattice.to(dev)
    sw = simplicial_workload("geom")
    N = sw.q.shape[2]
    pad = (torch.arange(N)[None, :] >= sw.counts[:, None]).to(dev)
    coords = (torch.randn(pad.shape[0], N, 3, generator=torch.Generator().manual_seed(5)) * 2.0 ** 0.5).to(dev)
    cases = (("c4_periodic_cells", PeriodicGeometryAdapter(pbc_radius=1).to(dev), (frac, None, lat),
              {"radius_cutoff": rw.cutoff}),
             ("c2_geom_molecules", NonPeriodicGeometryAdapter().to(dev), (coords, pad), {}))
    res = {}
    with torch.no_grad():
        for name, adapter, args, kw in cases:
            B, n = args[0].shape[:2]
            ms = _graph_ms(lambda: adapter(*args, **kw), per_graph=10, replays=5)  # noqa: B023
            nbytes = B * n * n * 6 * 4 + (B * n * ((n + 31) // 32) * 4 if kw else 0)
            gbs = nbytes / (ms * 1e-3) / 1e9
            res[name] = {"ms": round(ms, 5), "batch": B, "atoms": n, "output_bytes": nbytes,
                         "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                      "frac": round(gbs / HBM_PEAK_GBS, 4)}}
    return res


def measure_pair_mlp() -> dict:
    """The factorized geometry bias (SimplicialGeometryBias's u, v, w pairwise MLPs, mf_pair_mlp_bias) on
    configs[1]'s GEOM molecules: hidden 128, 16 rbf, 8 heads, from the non-periodic adapter's features;
    graph-replayed kernel time against the HBM roofline of its fp32 outputs (3 x [B, H, N, N]) and inputs."""
    import torch

    from matterformer_amd import pair_mlp
    from matterformer_amd.geometry import NonPeriodicGeometryAdapter
    from matterformer_amd.geometry_bias import SimplicialGeometryBias
    from matterformer_amd.workloads import simplicial_workload

    dev = torch.device("cuda", 0)
    sw = simplicial_workload("geom")
    B, H, N = sw.q.shape[0], sw.q.shape[1], sw.q.shape[2]
    pad = torch.arange(N)[None, :] >= sw.counts[:, None]
    coords = torch.randn(B, N, 3, generator=torch.Generator().manual_seed(5)) * 2.0 ** 0.5
    torch.manual_seed(6)
    module = SimplicialGeometryBias(H, mode="factorized", edge_bias_hidden_dim=128, edge_bias_n_rbf=16)
    with torch.no_grad():
        feats = NonPeriodicGeometryAdapter()(coords[:1], pad[:1])
        module._compute_factorized_terms(feats)  # materialises the LazyLinear layers (CPU, torch formulation)
        module = module.to(dev)
        feats = NonPeriodicGeometryAdapter().to(dev)(coords.to(dev), pad.to(dev))
        if not pair_mlp.serves(module, feats):
            raise RuntimeError("mf_pair_mlp_bias does not serve the bench configuration")
        ms = _graph_ms(lambda: pair_mlp.factorized_terms(module, feats), per_graph=10, replays=5)
    hidden = 128
    valid = int((sw.counts.long() ** 2 - sw.counts.long()).sum())
    nbytes = 3 * B * H * N * N * 4 + B * N * N * (4 * 4 + 1)
    gbs = nbytes / (ms * 1e-3) / 1e9
    flops = valid * 2 * (2 * (19 * hidden + hidden * H) + (16 * hidden + hidden * H))

    # a training step through the MLPs: forward, a loss over u, v, w, backward to the 12 weights
    # (mf_pair_mlp_bias_bwd through the autograd Function), against the same step on the torch formulation
    gen = torch.Generator().manual_seed(8)
    ups = [torch.randn(B, H, N, N, generator=gen).to(dev) for _ in range(3)]
    params = [p for m in (module.spoke_bias_u_mlp, module.spoke_bias_v_mlp, module.pair_bias_w_mlp)
              for p in m.parameters()]

    def train_kernel():
        u, v, w = module._compute_factorized_terms(feats)
        torch.autograd.grad((u * ups[0]).sum() + (v * ups[1]).sum() + (w * ups[2]).sum(), params)

    def train_torch():
        spoke, pairf = module._build_spoke_features(feats), module._build_pair_features(feats)
        mask = feats.pair_mask[:, None].float()
        u, v, w = (module._zero_pairwise_diag(mlp(f).permute(0, 3, 1, 2).contiguous()) * mask
                   for mlp, f in ((module.spoke_bias_u_mlp, spoke), (module.spoke_bias_v_mlp, spoke),
                                  (module.pair_bias_w_mlp, pairf)))
        torch.autograd.grad((u * ups[0]).sum() + (v * ups[1]).sum() + (w * ups[2]).sum(), params)

    if not pair_mlp.serves(module, feats):
        raise RuntimeError("mf_pair_mlp_bias_bwd does not serve the bench configuration")
    train_ms, _ = timed_loop(torch.cuda.current_stream(), train_kernel, 10, 3)
    torch_ms, _ = timed_loop(torch.cuda.current_stream(), train_torch, 3, 1)
    return {"ms": round(ms, 5), "batch": B, "atoms": N, "heads": H, "hidden": hidden, "rbf": 16,
            "valid_pairs": valid, "bytes": nbytes, "valid_gflop": round(flops / 1e9, 3),
            "valid_tflops_fp32": round(flops / (ms * 1e-3) / 1e12, 2),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4)},
            "train_step_ms": round(train_ms, 4), "train_step_torch_ms": round(torch_ms, 4),
            "train_step": "forward + loss over u, v, w + backward to the MLP weights (mf_pair_mlp_bias_bwd), "
                          "eager; torch: the same step on the torch formulation on the GPU"}


def measure_trunk() -> dict:
    """12-layer alternating trunk forward, bf16 weights and activations, 64 GEOM molecules."""
    import torch

    from matterformer_amd.trunk import AlternatingTrunk, TokenPacking
    from matterformer_amd.workloads import trunk_workload

    dev = torch.device("cuda", 0)
    w = trunk_workload()
    torch.manual_seed(4)
    trunk = AlternatingTrunk(w.d_model, w.heads, w.layers, knn_k=w.knn_k).to(dev).to(torch.bfloat16).eval()
    gen = torch.Generator().manual_seed(104)
    for blk in trunk.blocks:  # non-zero adaLN gates (the reference zero-initialises them)
        lin = blk.ada_ln[-1]
        lin.weight.data.copy_((torch.randn(lin.weight.shape, generator=gen) * 0.05).to(lin.weight.dtype))
        lin.bias.data.copy_((torch.randn(lin.bias.shape, generator=gen) * 0.05).to(lin.bias.dtype))
    x, cond = w.x.to(dev, torch.bfloat16), w.cond.to(dev, torch.bfloat16)
    coords, pad = w.coords.to(dev), w.pad_mask.to(dev)

    packing = TokenPacking(pad)

    def eager_padded():
        trunk.pack_tokens = False
        with torch.no_grad():
            trunk(x, cond, coords, pad)
        trunk.pack_tokens = True

    def eager_packed():
        with torch.no_grad():
            trunk(x, cond, coords, pad)

    def packed_step():
        with torch.no_grad():
            trunk(x, cond, coords, pad, packing=packing)

    stream = torch.cuda.current_stream()
    padded_ms, _ = timed_loop(stream, eager_padded, 10, 3)
    eager_ms, _ = timed_loop(stream, eager_packed, 10, 3)
    ms = graph_times(stream, packed_step, per_graph=1, replays=20)
    flops = w.valid_flops()
    atoms = int(w.counts.sum())
    return {"ms": round(ms, 4), "molecules_per_s": round(w.x.shape[0] / (ms * 1e-3), 1),
            "atoms_per_s": round(atoms / (ms * 1e-3), 1), "valid_gflop": round(flops["total"] / 1e9, 3),
            "valid_tflops": round(flops["total"] / (ms * 1e-3) / 1e12, 3),
            "gflop_split": {k: round(v / 1e9, 3) for k, v in flops.items() if k != "total"},
            "ms_source": "HIP events around replays of the packed forward captured in one HIP graph",
            "eager_packed_ms": round(eager_ms, 4), "eager_padded_ms": round(padded_ms, 4),
            "tokens_valid": packing.tokens, "tokens_padded": int(pad.numel()),
            "config": "12 layers d=512 H=8 MLP 4x, even simplicial (bf16_tc) / odd kNN-local k=32, bf16, "
                      "64 GEOM molecules padded to 181, seed 4, forward incl. kNN lists and masks; "
                      "per-token work on the valid atoms (TokenPacking)"}


def measure_trunk_geometry() -> dict:
    """configs[4] with the geometry terms: the trunk of measure_trunk plus a NonPeriodicGeometryAdapter and a
    SimplicialGeometryBias (factorized, hidden 128, 16 rbf; fp32 modules, output layers drawn N(0, 0.3^2) so
    the bias is not zero) whose features, u/v/w MLPs (mf_pair_mlp_bias) and noise gate run once per forward
    on the packing's compact layout and feed the six simplicial blocks through the pair kernel's bias K step."""
    import torch

    from matterformer_amd.geometry import NonPeriodicGeometryAdapter
    from matterformer_amd.geometry_bias import SimplicialGeometryBias
    from matterformer_amd.trunk import AlternatingTrunk, TokenPacking
    from matterformer_amd.workloads import trunk_workload

    dev = torch.device("cuda", 0)
    w = trunk_workload()
    torch.manual_seed(4)
    bias = SimplicialGeometryBias(w.heads, mode="factorized", edge_bias_hidden_dim=128, edge_bias_n_rbf=16)
    trunk = AlternatingTrunk(w.d_model, w.heads, w.layers, knn_k=w.knn_k,
                             geometry_adapter=NonPeriodicGeometryAdapter(), simplicial_geometry_bias=bias)
    x, cond = w.x.to(dev, torch.bfloat16), w.cond.to(dev, torch.bfloat16)
    coords, pad = w.coords.to(dev), w.pad_mask.to(dev)
    gen = torch.Generator().manual_seed(105)
    sigma = (torch.rand(w.x.shape[0], generator=gen) * 2.0 + 0.05).to(dev)
    with torch.no_grad():
        # materialises the LazyLinear layers (CPU, torch formulation)
        bias._compute_factorized_terms(NonPeriodicGeometryAdapter()(w.coords[:1], w.pad_mask[:1]))
        for name, prm in bias.named_parameters():
            if name.endswith(".2.weight") or name.endswith(".2.bias"):
                prm.data.copy_(torch.randn(prm.shape, generator=gen) * 0.3)
    trunk.blocks.to(dev).to(torch.bfloat16)
    trunk.geometry_adapter.to(dev)
    bias.to(dev)
    trunk.eval()
    for blk in trunk.blocks:
        lin = blk.ada_ln[-1]
        lin.weight.data.copy_((torch.randn(lin.weight.shape, generator=gen) * 0.05).to(lin.weight.dtype))
        lin.bias.data.copy_((torch.randn(lin.bias.shape, generator=gen) * 0.05).to(lin.bias.dtype))
    packing = TokenPacking(pad)

    def step():
        with torch.no_grad():
            trunk(x, cond, coords, pad, sigma=sigma, packing=packing)

    stream = torch.cuda.current_stream()
    eager_ms, _ = timed_loop(stream, step, 10, 3)
    ms = graph_times(stream, step, per_graph=1, replays=20)
    return {"ms": round(ms, 4), "molecules_per_s": round(w.x.shape[0] / (ms * 1e-3), 1),
            "eager_ms": round(eager_ms, 4),
            "ms_source": "HIP events around replays of the packed forward captured in one HIP graph",
            "config": "the c5_trunk configuration plus NonPeriodicGeometryAdapter + SimplicialGeometryBias "
                      "(factorized, fp32), sigma U[0.05, 2.05), terms on the compact layout"}


# The reference's module benchmark grid (d_model, heads, tokens, batch): scripts/benchmark_simplicial_attention.py:27-42
MODULE_GRID = (
    (512, 8, 24, 256), (512, 8, 32, 128), (512, 8, 48, 64), (512, 8, 64, 32), (512, 8, 96, 16), (512, 8, 128, 8),
    (512, 8, 192, 4), (768, 12, 24, 256), (768, 12, 32, 128), (768, 12, 48, 64), (768, 12, 64, 32),
    (768, 12, 96, 16), (768, 12, 128, 8), (768, 12, 192, 4),
)


def _module_case(impl, mode, pass_type, d_model, heads, tokens, batch, *, pad=None, warmup=2, iters=5):
    """One case run as the reference harness does (scripts/benchmark_simplicial_attention.py:167-259): the
    module in eval (forward, no_grad) or train mode (out.square().mean() backward), inputs drawn inside every
    run (randn x and, for mode "factorized", randn u, v, w, gate), host clock around iters runs after warmup.
    `pad` (True = padding, [batch, tokens]) replaces the all-valid mask of the reference grid."""
    import torch

    from matterformer_amd.simplicial_attention import TwoSimplicialAttention
    from matterformer_amd.simplicial_types import SimplicialAttentionMask, SimplicialFactorizedBias

    dev = torch.device("cuda", 0)
    dt = torch.bfloat16
    torch.manual_seed(0)
    attn = TwoSimplicialAttention(dim=d_model, num_heads=heads, chunk_size=min(tokens, 128), dropout=0.0,
                                  impl=impl, precision="bf16_tc").to(device=dev, dtype=dt)
    attn.eval() if pass_type == "forward" else attn.train()
    mask = SimplicialAttentionMask.from_key_padding_mask(pad, batch_size=batch, num_tokens=tokens, device=dev)

    def run_once():
        rg = pass_type == "train_step"
        x = torch.randn(batch, tokens, d_model, device=dev, dtype=dt, requires_grad=rg)
        fb = None
        if mode == "factorized":
            fb = SimplicialFactorizedBias(*(torch.randn(batch, heads, tokens, tokens, device=dev, dtype=dt,
                                                        requires_grad=rg) for _ in range(3)),
                                          torch.randn(batch, heads, tokens, device=dev, dtype=dt, requires_grad=rg))
        attn.zero_grad(set_to_none=True)
        if pass_type == "forward":
            with torch.no_grad():
                attn(x, attention_mask=mask, factorized_bias=fb)
            return
        attn(x, attention_mask=mask, factorized_bias=fb).square().mean().backward()

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run_once()
    torch.cuda.synchronize()
    first_ms = (time.perf_counter() - t0) * 1e3
    for _ in range(warmup):
        run_once()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    t0 = time.perf_counter()
    for _ in range(iters):
        run_once()
    torch.cuda.synchronize()
    steady_ms = (time.perf_counter() - t0) * 1e3 / iters
    return {"impl": impl, "mode": mode, "pass": pass_type, "d_model": d_model, "heads": heads, "tokens": tokens,
            "batch": batch, "first_ms": round(first_ms, 3), "steady_ms": round(steady_ms, 4),
            "peak_mem_mib": round(torch.cuda.max_memory_allocated(dev) / 2**20, 1),
            "last_impl_used": getattr(attn, "_last_impl_used", None)}


def measure_module_c2() -> dict:
    """SimplicialAttention(512, 8) with impl="hip" on C2's batch (64 GEOM molecules padded to 181, their key
    padding mask): forward and train step, the reference harness's timing (inputs drawn per run)."""
    from matterformer_amd.workloads import simplicial_workload

    w = simplicial_workload("geom")
    pad = (~w.pair_key_valid).to("cuda")
    B, N = pad.shape
    res = {}
    for pass_type in ("forward", "train_step"):
        for mode in ("none", "factorized"):
            c = _module_case("hip", mode, pass_type, 512, 8, N, B, pad=pad, warmup=3, iters=10)
            res[f"{pass_type}_{mode}_ms"] = c["steady_ms"]
            res[f"{pass_type}_{mode}_impl"] = c["last_impl_used"]
    res["molecules_per_s_forward"] = round(B / (res["forward_none_ms"] * 1e-3), 1)
    res["config"] = ("TwoSimplicialAttention(dim=512, num_heads=8, impl='hip', bf16_tc), x [64, 181, 512] bf16, "
                     "C2 key padding mask; per run: randn inputs (and u, v, w, gate for 'factorized'), "
                     "in_proj -> attention -> out_proj (train step: + backward of out.square().mean())")
    return res


def bench_module(args) -> int:
    """The reference harness's grid through the mirrored module: impl hip and torch, modes none / factorized,
    forward and train step (one JSON line; `value` = geometric mean of the hip forward, mode none)."""
    import math

    cases = []
    for (d, h, t, b) in MODULE_GRID:
        for pass_type in ("forward", "train_step"):
            for mode in ("none", "factorized"):
                for impl in ("hip", "torch"):
                    cases.append(_module_case(impl, mode, pass_type, d, h, t, b))
                    print(json.dumps({"case": cases[-1]}), file=sys.stderr, flush=True)
    fwd = [c["steady_ms"] for c in cases if c["impl"] == "hip" and c["pass"] == "forward" and c["mode"] == "none"]
    gm = math.exp(sum(math.log(x) for x in fwd) / len(fwd))
    line = _line("TwoSimplicialAttention module forward steady ms, reference harness grid (geometric mean)",
                 round(gm, 4), "ms", gm, args, "bf16", "synthetic (randn per run, as the reference harness)",
                 {"workload": "scripts/benchmark_simplicial_attention.py grid, bf16_tc, all tokens valid",
                  "grid": [list(g) for g in MODULE_GRID]}, cases=cases)
    line["higher_is_better"] = False
    print(json.dumps(line), flush=True)
    return 0


def _line(metric, value, unit, ms, args, dtype, data, config, **more):
    line = {"metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": dtype, "data": data, "config": config}
    line.update(more)
    return line


def bench_knn(args) -> int:
    m = measure_knn(args.cpu_sample)
    print(json.dumps(_line("kNN top-16 queries/s (configs[2] scaled to 32768 molecules)", m["queries_per_s"],
                           "queries/s", m["scaled_ms"], args, "f32", "synthetic (seeded, BASELINE.json configs[2])",
                           {"workload": "kNN top-16, 181 atoms/molecule, coords N(0, 2 A^2)",
                            "batch": m["scaled_batch"], "atoms": 181, "k": 16, "c3_batch32_ms": m["c3_ms"]},
                           roofline=m["roofline"], cpu_baseline=m["cpu_baseline"])), flush=True)
    return 0


def bench_radius(args) -> int:
    m = measure_radius(args.cpu_sample)
    print(json.dumps(_line("radius mask + radius attention cells/s (configs[3])", m["cells_per_s"], "cells/s",
                           m["step_ms"], args, "bf16", "synthetic (seeded, BASELINE.json configs[3])",
                           {"workload": "periodic MOF cells, 6 A cutoff, minimum image, 64-atom tiles",
                            "cells": m["cells"], "atoms": m["atoms"], "allowed_pairs": m["allowed_pairs"],
                            "mask_ms": m["mask_ms"], "attn_ms": m["attn_ms"]},
                           roofline=m["roofline"], cpu_baseline=m["cpu_baseline"])), flush=True)
    return 0


def bench_trunk(args) -> int:
    m = measure_trunk()
    print(json.dumps(_line("configs[4] trunk forward molecules/s", m["molecules_per_s"], "molecules/s", m["ms"], args,
                           "bf16", "synthetic (seeded, BASELINE.json configs[4]); random-init weights",
                           {"workload": m["config"]}, atoms_per_s=m["atoms_per_s"],
                           valid_tflops=m["valid_tflops"], gflop_split=m["gflop_split"])), flush=True)
    return 0


def _simplicial_call(lib, ops, qv, pkv, dtype_code, precision, out=None, out_f32=None, lse=None, bias=None):
    """A step closure calling mf_simplicial_fwd on torch's current stream (so graph capture records it)."""
    import torch

    from matterformer_amd import _native

    B, H, N, D = ops[0].shape
    ws_bytes = lib.mf_simplicial_fwd_workspace_size(B, H, N, D, dtype_code)
    ws = torch.zeros(max(int(ws_bytes), 16), dtype=torch.uint8, device=ops[0].device)
    extra = {}
    if bias is not None:
        extra = dict(bias_u=bias[0].data_ptr(), bias_v=bias[1].data_ptr(), bias_w=bias[2].data_ptr(),
                     bias_gate=bias[3].data_ptr(), bias_dtype=_native.dtype_code(bias[0].dtype))
    a = _native.MfSimplicialFwdArgs(
        q=ops[0].data_ptr(), k1=ops[1].data_ptr(), v1=ops[2].data_ptr(), k2=ops[3].data_ptr(), v2=ops[4].data_ptr(),
        query_valid=qv.data_ptr(), pair_key_valid=pkv.data_ptr(), pair_valid=None,
        out=_native.ptr(out), out_f32=_native.ptr(out_f32), lse=_native.ptr(lse),
        workspace=ws.data_ptr(), workspace_bytes=ws.numel(), batch=B, heads=H, tokens=N, head_dim=D,
        dtype=dtype_code, precision=_native.MF_PREC[precision], **extra)
    fwd = lib.mf_simplicial_fwd

    def step():
        st = fwd(a, torch.cuda.current_stream().cuda_stream)
        if st != 0:
            raise RuntimeError(f"mf_simplicial_fwd failed: {_native.last_error()}")

    step.keepalive = (a, ws, ops, out, out_f32, lse, bias)
    return step


def measure_simplicial_extras(lib, w, wd) -> dict:
    """Training-state forward, forward + backward, factorized bias (C2), and C1 fp32."""
    import torch

    from matterformer_amd import _native
    from matterformer_amd.hip_simplicial_attention import hip_simplicial_attention_backward
    from matterformer_amd.workloads import simplicial_workload

    dev = wd.q.device
    B, H, N, D = wd.shape
    ops = [t.contiguous() for t in (wd.q, wd.k1, wd.v1, wd.k2, wd.v2)]
    fwd_flops = w.valid_flops()
    out = torch.empty(B, H, N, D, dtype=torch.bfloat16, device=dev)
    out32 = torch.empty(B, H, N, D, dtype=torch.float32, device=dev)
    lse = torch.empty(B, H, N, dtype=torch.float32, device=dev)
    train_step = _simplicial_call(lib, ops, wd.query_valid, wd.pair_key_valid, _native.MF_DTYPE_BF16, "bf16_tc",
                                  out=out, out_f32=out32, lse=lse)
    train_ms = _graph_ms(train_step)
    res = {"train_state_fwd": {"ms": round(train_ms, 5), "tflops": round(fwd_flops / (train_ms * 1e-3) / 1e12, 3),
                               "outputs": "bf16 out + fp32 out + fp32 lse (the reference launcher's contract)"}}

    # backward: mf_simplicial_bwd on the training-state outputs
    gen = torch.Generator().manual_seed(11)
    go = torch.randn(B, H, N, D, generator=gen).to(dev, torch.bfloat16)
    train_step()
    torch.cuda.synchronize()

    def bwd_step():
        hip_simplicial_attention_backward(go, *ops, out32, lse, query_valid=wd.query_valid,
                                          pair_key_valid=wd.pair_key_valid, pair_valid=None, precision="bf16_tc")

    bwd_step()
    bwd_eager_ms, _ = timed_loop(torch.cuda.current_stream(), bwd_step, 10, 2)
    bwd_ms = _graph_ms(bwd_step, per_graph=10, replays=5)
    bwd_flops = 3 * fwd_flops  # dP, dq, dk1, dk2, dv1, dv2: 12 D n^3 per head against the forward's 4 D n^3
    res["fwd_bwd"] = {
        "fwd_ms": round(train_ms, 5), "bwd_ms": round(bwd_ms, 5), "ms": round(train_ms + bwd_ms, 5),
        "molecules_per_s": round(B / ((train_ms + bwd_ms) * 1e-3), 1),
        "valid_gflop": round(4 * fwd_flops / 1e9, 3),
        "bwd_roofline": {"bound": "mfma", "achieved": round(bwd_flops / (bwd_ms * 1e-3) / 1e12, 3),
                         "peak": BF16_DENSE_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(bwd_flops / (bwd_ms * 1e-3) / 1e12 / BF16_DENSE_PEAK_TFLOPS, 5),
                         "kernel": "mf::pbwd::pair_bwd_kernel (pairs as keys, fp16 operands, LPT plan, large "
                                   "molecules in two halves) with its plan, combine and zero-rows launches; "
                                   "deterministic, no atomics",
                         "kernel_ms": round(bwd_ms, 5),
                         "note": "hip_simplicial_attention_backward graph-replayed, bf16 gradients written by the "
                                 "kernels (no fill, no cast); eager call " + f"{bwd_eager_ms:.4f} ms"},
    }

    # factorized bias (bf16), the default trunk's call: the pair kernel with the bias K step
    bias = [(torch.randn(B, H, N, N, generator=gen) * 0.5).to(dev, torch.bfloat16) for _ in range(3)] + \
           [torch.randn(B, H, N, generator=gen).to(dev, torch.bfloat16)]
    bias_step = _simplicial_call(lib, ops, wd.query_valid, wd.pair_key_valid, _native.MF_DTYPE_BF16, "bf16_tc",
                                 out=out, bias=bias)
    bias_ms = _graph_ms(bias_step)
    res["bias_fwd"] = {"ms": round(bias_ms, 5), "tflops": round(fwd_flops / (bias_ms * 1e-3) / 1e12, 3),
                       "kernel": "mf::spair::simplicial_pair_kernel<bf16, 64, pair_valid=0, bias=1> "
                                 "(factorized bias, bf16)"}
    # its backward: the bias training state, then mf_simplicial_bwd with the nine gradients
    bias_state = _simplicial_call(lib, ops, wd.query_valid, wd.pair_key_valid, _native.MF_DTYPE_BF16, "bf16_tc",
                                  out=out, out_f32=out32, lse=lse, bias=bias)
    bias_state()
    torch.cuda.synchronize()

    def bias_bwd_step():
        hip_simplicial_attention_backward(go, *ops, out32, lse, query_valid=wd.query_valid,
                                          pair_key_valid=wd.pair_key_valid, pair_valid=None, precision="bf16_tc",
                                          u=bias[0], v_bias=bias[1], w=bias[2], gate=bias[3])

    bias_bwd_step()
    bias_bwd_eager_ms, _ = timed_loop(torch.cuda.current_stream(), bias_bwd_step, 10, 2)
    bias_bwd_ms = _graph_ms(bias_bwd_step, per_graph=10, replays=5)
    res["bias_bwd"] = {"ms": round(bias_bwd_ms, 5), "eager_ms": round(bias_bwd_eager_ms, 5),
                       "kernel": "mf::pbwd::pair_bwd_kernel<bias=1> (query tiles in passes of at most three) with "
                                 "its plan, combine, bias finish and clearing launches; dq, dk1, dv1, dk2, dv2, du, "
                                 "dv_bias, dw, dgate in bf16, written in full"}

    # C1: QM9 fp32
    c1 = simplicial_workload("qm9").to(dev)
    c1_ops = [t.contiguous() for t in (c1.q, c1.k1, c1.v1, c1.k2, c1.v2)]
    c1_out = torch.empty_like(c1_ops[0])
    c1_step = _simplicial_call(lib, c1_ops, c1.query_valid, c1.pair_key_valid, _native.MF_DTYPE_F32, "ieee_fp32",
                               out=c1_out)
    c1_ms = _graph_ms(c1_step)
    c1_flops = c1.valid_flops()
    res["c1_qm9_fp32"] = {"ms": round(c1_ms, 5), "tflops": round(c1_flops / (c1_ms * 1e-3) / 1e12, 3),
                          "molecules_per_s": round(c1.q.shape[0] / (c1_ms * 1e-3), 1),
                          "roofline": {"bound": "mfma", "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                                       "frac": round(c1_flops / (c1_ms * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS, 5)}}
    return res


def main() -> int:
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}, WORLD_SIZE {world}); "
              "every kernel here works per molecule or per cell with no cross-GPU exchange: data "
              "parallelism over molecules or cells shards the path without any forward exchange.",
              file=sys.stderr)
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
    if args.workload == "trunk":
        return bench_trunk(args)
    if args.workload == "module":
        return bench_module(args)
    dev = torch.device("cuda", 0)
    lib = _native.lib()

    w = simplicial_workload("geom")
    wd = w.to(dev, torch.bfloat16)
    B, H, N, D = wd.shape
    ops = [t.contiguous() for t in (wd.q, wd.k1, wd.v1, wd.k2, wd.v2)]
    out = torch.empty((B, H, N, D), device=dev, dtype=torch.bfloat16)
    step = _simplicial_call(lib, ops, wd.query_valid, wd.pair_key_valid, _native.MF_DTYPE_BF16, "bf16_tc", out=out)
    stream = torch.cuda.current_stream(dev)

    ms_per_step, wall = timed_loop(stream, step, args.steps, args.warmup)

    flops = w.valid_flops()
    tflops = flops / (ms_per_step * 1e-3) / 1e12
    atoms = int(w.counts.sum())

    # kernel duration: graph of 20 back-to-back launches, replayed; plus single-launch events for reference
    kernel_ms = graph_times(stream, step)
    single_ms, _ = event_times(stream, step, 100)
    achieved = flops / (kernel_ms * 1e-3) / 1e12

    extra = None
    if not args.no_extra:
        extra = measure_simplicial_extras(lib, w, wd)
        extra["knn"] = measure_knn(args.cpu_sample)
        extra["radius"] = measure_radius(args.cpu_sample)
        extra["c5_trunk"] = measure_trunk()
        extra["c5_trunk_geometry"] = measure_trunk_geometry()
        extra["geometry_features"] = measure_geometry()
        extra["pair_mlp_bias"] = measure_pair_mlp()
        extra["module_c2"] = measure_module_c2()

    cpu = cpu_baseline(w, args.cpu_sample, args.cpu_threads) if args.cpu_sample > 0 else None

    line = _line(
        "2-simplicial attn fwd TFLOP/s (%MFMA peak) + molecules/s, GEOM-Drugs shape", round(tflops, 3), "TFLOP/s",
        ms_per_step, args, "bf16", "synthetic (seeded, BASELINE.json configs[1])",
        {"workload": "GEOM-Drugs-like 2-simplicial attention fwd (configs[1])", "batch": B, "heads": H,
         "tokens_padded": N, "head_dim": D, "valid_atoms": atoms, "valid_gflop": round(flops / 1e9, 4)},
        pct_mfma_peak=round(100.0 * tflops / BF16_DENSE_PEAK_TFLOPS, 3),
        molecules_per_s=round(B / (ms_per_step * 1e-3), 1),
        atoms_per_s=round(atoms / (ms_per_step * 1e-3), 1),
        wall_s=round(wall, 4),
        roofline={
            "bound": "mfma", "achieved": round(achieved, 3), "peak": BF16_DENSE_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / BF16_DENSE_PEAK_TFLOPS, 5), "traffic": committed_traffic("simplicial_fwd_geom"),
            "kernel": "mf_simplicial_fwd launch: simplicial_pair_kernel<bf16, 64, pair_valid=0>",
            "kernel_ms": round(kernel_ms, 5), "kernel_ms_source": "HIP events around replays of a 20-launch graph",
            "single_launch_event_ms": round(single_ms, 5),
        },
        cpu_baseline=cpu,
        extra=extra,
    )
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
