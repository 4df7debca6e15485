"""Build librte_hip.so (gfx950) in-tree with hipcc.

Usage: python speedup-thingy_amd/build.py [--jobs N]
The shared library lands next to the Python package (rte_amd/librte_hip.so) so
it travels with the source tree; no JIT cache, no site-packages install.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OUT = HERE / "rte_amd" / "librte_hip.so"
OBJ = HERE / "_build"
SOURCES = ["gemm.hip", "route.hip", "norm.hip", "loss.hip", "shortlist.hip", "segreduce.hip", "glue.hip", "distill.hip", "macro.hip", "macro_fused.hip", "macro_cons.hip", "adamw.hip", "attention.hip", "noalloc.hip", "dispatch.hip", "svdsel.hip", "svd_fused.hip", "router.hip", "bookkeep.hip", "f32.hip", "replay.hip", "pool_fused.hip", "capi.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # packed fp32 ops are kept out of the device code on purpose
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the ROCm toolchain is required to build librte_hip")


def _compile(src: Path, obj: Path) -> None:
    cmd = [_hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr[-6000:]}")


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    OBJ.mkdir(exist_ok=True)
    objs = [OBJ / (Path(s).stem + ".o") for s in SOURCES]
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        futs = [pool.submit(_compile, CSRC / s, o) for s, o in zip(SOURCES, objs)]
        for f in futs:
            f.result()
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [_hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr[-6000:]}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args(argv)
    build(args.jobs, verbose=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
