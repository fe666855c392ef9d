"""Builds the native library ``libopake_amd.so`` for gfx950 in-tree.

Every ``opake_amd/csrc/*.hip`` file is compiled with ``hipcc`` for gfx950
(packed-fp32 instruction forms disabled) and linked into one shared library
next to this file.  Nothing here runs at import time.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
LIB_PATH = PKG_DIR / "libopake_amd.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; ROCm is required to build opake_amd")
    return path


def _compile(src: Path, obj: Path) -> None:
    cmd = [_hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")


def build_native(verbose: bool = False) -> Path:
    """Compile all HIP sources and link ``libopake_amd.so``; returns its path."""
    objdir = PKG_DIR / "_build"
    objdir.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    objs = [objdir / (s.stem + ".o") for s in sources]
    workers = min(len(sources), max(1, (os.cpu_count() or 2)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(lambda so: _compile(*so), zip(sources, objs)))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build_native(verbose=True)
