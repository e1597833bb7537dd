"""Build the CPU oracle library (test infrastructure only).

``python -m oracle.build`` (or ``build()``) compiles ``scan_ref.c`` with gcc into
``oracle/liboracle_scan.so``.  The reference (createcentury/mamba-metal) has no
C/C++ sources for this path -- its kernels are Metal Shading Language bodies
JIT-compiled by MLX -- so there is no ``oracle/_ref`` build: the reference is
unbuildable here and the oracle is this restatement, pinned by the checks in
``tests/test_oracle.py``.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "scan_ref.c"
LIB = HERE / "liboracle_scan.so"

# -ffp-contract=off keeps the float arithmetic un-fused (numpy-like); -mavx2/-mfma
# target any x86-64-v3 host (the GPU box host may differ from this container).
CFLAGS = ["-O3", "-fPIC", "-shared", "-fopenmp", "-ffp-contract=off", "-mavx2", "-mfma", "-std=c11"]


def build(verbose: bool = False) -> Path:
    tmp = LIB.with_suffix(".so.tmp")
    cmd = ["gcc", *CFLAGS, str(SRC), "-o", str(tmp), "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(LIB)
