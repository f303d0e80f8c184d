"""Build libmlxr_moe.so (the C-ABI library of HIP kernels) for gfx950.

Compiles every source under csrc/ with hipcc into _build/ (in parallel),
then links mlx-rs_amd/libmlxr_moe.so in-tree so that it travels with the
repository snapshot.  Always recompiles: `build()` is the "does it build"
check.

    python mlx-rs_amd/build.py [--jobs N]
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
BUILD = HERE / "_build"
LIB = HERE / "libmlxr_moe.so"
ARCH = "gfx950"

SOURCES = [
    "quant.hip",
    "router.hip",
    "dispatch.hip",
    "qgemm.hip",
    "prefill.hip",
    "combine.hip",
    "nn.cpp",
    "profile.cpp",
    "capi.cpp",
    "noalloc.hip",
    "probe.hip",
]

COMMON = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # packed fp32 VALU ops stay off on this hardware pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # every multiply and add rounds separately unless the source calls fmaf
    # (hipcc's default would fuse them): the combine and softmax then match
    # a plain C evaluation of the same expressions bit for bit
    "-ffp-contract=off",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libmlxr_moe.so)")


def _compile(src: str) -> Path:
    obj = BUILD / (src.replace(".", "_") + ".o")
    cmd = [hipcc(), *COMMON, "-c", str(CSRC / src), "-o", str(obj)]
    if src.endswith(".hip"):
        cmd[1:1] = ["-x", "hip"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    build(args.jobs, verbose=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
