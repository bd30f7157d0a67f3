"""Build recipe for the oracle's C restatement (test infrastructure only).

``python -m oracle.build`` compiles oracle/ckv_oracle.c with gcc into
oracle/_build/libckv_oracle.so. -ffp-contract=off keeps every fp32 product and sum separately
rounded, as the reference's torch ops are. The reference itself is pure Python (no C/C++
sources), so there is no oracle/_ref build.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SRC = HERE / "ckv_oracle.c"
OUT_DIR = HERE / "_build"
LIB = OUT_DIR / "libckv_oracle.so"
CFLAGS = ["-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-Wall", "-Wextra"]


def build(verbose: bool = False) -> Path:
    OUT_DIR.mkdir(exist_ok=True)
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [os.environ.get("CC", "gcc"), *CFLAGS, str(SRC), "-o", str(tmp), "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("oracle build failed")
    if res.stderr and verbose:
        sys.stderr.write(res.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
