"""Build libanima_hip.so in-tree with hipcc for gfx950.

``python -m animaxs_amd.build`` (or ``animaxs_amd.build.build()``) compiles every
``csrc/*.hip`` with ``hipcc --offload-arch=gfx950`` and every ``csrc/*.cpp`` with
``g++``, then links ``animaxs_amd/libanima_hip.so``.  Packed-FP32 instruction
selection is disabled for all device code.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
OUT = PKG / "libanima_hip.so"
OBJ = PKG / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}", f"-I{CSRC}",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", f"-I{INCLUDE}", f"-I{CSRC}"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")


def _compile(src: Path) -> Path:
    obj = OBJ / (src.name + ".o")
    if src.suffix == ".hip":
        _run([HIPCC, "-x", "hip", "-c", str(src), "-o", str(obj), *HIP_FLAGS])
    else:
        _run([shutil.which("g++") or "g++", "-c", str(src), "-o", str(obj), *CXX_FLAGS])
    return obj


def build(verbose: bool = True, jobs: int | None = None) -> Path:
    """Compile all sources and link the shared library; returns its path."""
    OBJ.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    if not sources:
        raise RuntimeError(f"no sources in {CSRC}")
    jobs = jobs or min(8, len(sources), os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = OUT.with_suffix(".so.tmp")
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT} ({OUT.stat().st_size} bytes) from {len(sources)} sources")
    return OUT


if __name__ == "__main__":
    build()
    sys.exit(0)
