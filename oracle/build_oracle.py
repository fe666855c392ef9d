"""Builds the C oracle (TEST INFRASTRUCTURE) into oracle/_build/ with gcc.

The reference (JetBrains-Research/opake) is Python + Triton with no C/C++
sources on this path, so there is no ``oracle/_ref`` build: only this
restatement is compiled.
"""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "dpc_oracle.c"
OUT = HERE / "_build" / "libdpc_oracle.so"


def build_oracle() -> Path:
    OUT.parent.mkdir(exist_ok=True)
    cc = shutil.which("gcc") or "cc"
    cmd = [cc, "-O2", "-fPIC", "-shared", "-ffp-contract=off", str(SRC), "-o", str(OUT), "-lm"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}\n{res.stderr}")
    return OUT


if __name__ == "__main__":
    print(build_oracle())
