"""Build libkda_mi355x.so in-tree with hipcc for gfx950.

Usage: python kimi-k3-pytorch_amd/build_lib.py   (or __graft_entry__.build()).
Every .hip / .cpp file under csrc/ is compiled into one shared library placed
next to the Python package (kda/libkda_mi355x.so), where kda/_lib.py loads it.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
CSRC = HERE / "csrc"
INCLUDE = REPO / "include"
OUT = HERE / "kda" / "libkda_mi355x.so"
OBJ_DIR = HERE / "_build"

ARCH = "gfx950"
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
    # Packed FP32 VALU ops are not generated (device pass only; the host pass
    # warns that it does not know the feature).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # keep MFMA accumulators in ordinary VGPRs instead of round-tripping them
    # through AGPRs (the state-scan loop converts and rescales them every chunk)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; ROCm is required to build libkda_mi355x.so")
    return exe


def _compile(src: Path) -> Path:
    obj = OBJ_DIR / (src.name + ".o")
    cmd = [_hipcc(), *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    OBJ_DIR.mkdir(exist_ok=True)
    sources = sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=max(jobs, 1)) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} from {len(sources)} sources")
    return OUT


if __name__ == "__main__":
    build()
