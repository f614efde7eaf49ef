"""Build the gfx950 HIP library ``hi3d_amd/libhi3d_amd.so`` in-tree with hipcc.

Usage: ``python hi3dv1.0-mlx_amd/build.py`` (each source compiles in parallel, then one
link step). Every source is compiled with packed-fp32 instructions disabled.
"""

from __future__ import annotations

import concurrent.futures as futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
CSRC = HERE / "csrc"
OUT = HERE / "hi3d_amd" / "libhi3d_amd.so"
BUILD = HERE / "_build"

ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    "-Wno-unused-result",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build hi3d_amd")
    return path


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every ``csrc/*.hip`` for gfx950 and link ``libhi3d_amd.so``."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    workers = min(len(sources), max(1, (os.cpu_count() or 4)))
    with futures.ThreadPoolExecutor(workers) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
