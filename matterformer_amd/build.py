"""Build libmf_hip.so (the gfx950 kernels + C ABI) in-tree with hipcc.

Usage: ``python -m matterformer_amd.build`` (or ``build()`` from Python).
The library lands in ``matterformer_amd/_lib/libmf_hip.so``; it is git-ignored
but travels with the source tree.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC_DIR = PACKAGE_DIR / "csrc"
LIB_DIR = PACKAGE_DIR / "_lib"
LIB_PATH = LIB_DIR / "libmf_hip.so"
INCLUDE_DIR = PACKAGE_DIR.parent / "include"

OFFLOAD_ARCH = "gfx950"

# Common hipcc flags.  Packed fp32 VALU ops are disabled for all device code.
BASE_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE_DIR}",
]

# Sources whose floating-point results must match a CPU restatement bit for
# bit are built without FMA contraction.
PER_FILE_FLAGS = {
    "knn.hip": ["-ffp-contract=off"],
    "radius.hip": ["-ffp-contract=off"],
    "geometry.hip": ["-ffp-contract=off"],
    "token_rows.hip": ["-ffp-contract=off"],
    "pair_mlp.hip": ["-ffp-contract=off"],
    # The pair kernel's unit claim is one lane's atomicAdd whose result is
    # needed only after the unit's output is written.  The atomic optimizer
    # would rewrite it into a wave-wide form that reads the result at once,
    # so the output phase would wait out the atomic's round trip.
    "simplicial_pair.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: set HIPCC or install ROCm")


def _compile_one(hipcc: str, src: Path, obj: Path, verbose: bool) -> None:
    cmd = [hipcc, *BASE_FLAGS, *PER_FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = ("packed-fp32-ops", "not a recognized feature")
    err = "\n".join(line for line in proc.stderr.splitlines() if not any(n in line for n in noise))
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build(verbose: bool = False) -> Path:
    """Compile every ``csrc/*.hip`` for gfx950 and link ``libmf_hip.so``."""
    hipcc = _hipcc()
    sources = sorted(CSRC_DIR.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
    obj_dir = LIB_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    objs = [obj_dir / (src.stem + ".o") for src in sources]
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        futures = [pool.submit(_compile_one, hipcc, s, o, verbose) for s, o in zip(sources, objs)]
        for fut in futures:
            fut.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link of libmf_hip.so failed:\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
