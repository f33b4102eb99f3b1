"""Builds liblse_int8.so in-tree from csrc/*.hip with hipcc for gfx950.

Run as `python llm-serving-engine_amd/build_ext.py` or through `__graft_entry__.build()`. Every
call recompiles: the objects are cheap and a stale library is worse than a slow build.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_ROOT = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_ROOT / "include"
BUILD_DIR = PKG_DIR / "_build"
LIB_NAME = "liblse_int8.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

# Packed-fp32 VALU forms are kept out of every code object (the compiler would otherwise form
# them from plain float code); fp32 division and sqrt stay IEEE correctly rounded, which the
# bit-exact quantizers rely on.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the int8 Linear library needs ROCm's hipcc")
    return path


def _compile(src: Path, extra: list[str]) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIP_FLAGS, *extra, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stderr}")
    return obj


def build(extra_flags: list[str] | None = None, jobs: int | None = None) -> Path:
    """Compiles every csrc/*.hip and links LIB_PATH; returns its path."""
    extra = list(extra_flags or [])
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = jobs or min(len(sources), os.cpu_count() or 1, 8)
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(lambda s: _compile(s, extra), sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link of {LIB_NAME} failed:\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(sys.argv[1:]))
