"""Build recipe for the gfx950 KV-repair library (``chunkkv_amd/_lib/libchunkkv_amd.so``).

Run ``python -m chunkkv_amd.build``. hipcc cross-compiles for gfx950 without a GPU. The
library is a plain C-ABI shared object (see ``include/chunkkv_amd.h``); Python loads it with
ctypes after ``import torch`` so that it binds to the HIP runtime torch already loaded.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
LIB_DIR = PKG / "_lib"
LIB_NAME = "libchunkkv_amd.so"
SOURCES = ["abi.hip", "rerope_gather.hip", "assemble.hip", "deviation.hip", "select.hip", "select_gather.hip", "deviation_select.hip",
           "scatter.hip", "layer1_repair.hip", "attention.hip", "rope.hip", "extract.hip", "norm.hip"]
HOST_SOURCES = ["token_hash.cpp"]
ARCH = "gfx950"
GXX_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-pthread", "-Wall", "-Wextra"]

# -ffp-contract=off: products and sums stay separately rounded, like the reference's torch ops.
# -packed-fp32-ops disabled: no v_pk_*_f32 code generation (kept scalar fp32).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",  # MFMA accumulators in VGPRs (no accumulator-register copies)
    # the first 16 dwords of every kernel's arguments arrive in SGPRs at wave start instead of through
    # a scalar load (measured ~0.2 us less per short launch in a chain of them)
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found: install ROCm or set ROCM_PATH")
    return found


def lib_path() -> Path:
    return LIB_DIR / LIB_NAME


def build(verbose: bool = False) -> Path:
    """Compile every source for gfx950 and link the shared library. Always recompiles."""
    LIB_DIR.mkdir(exist_ok=True)
    obj_dir = LIB_DIR / "obj"
    obj_dir.mkdir(exist_ok=True)
    cc = hipcc()
    objs = []
    for src in SOURCES:
        obj = obj_dir / (Path(src).stem + ".o")
        cmd = [cc, *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(CSRC / src), "-o", str(obj)]
        _run(cmd, verbose)
        objs.append(str(obj))
    for src in HOST_SOURCES:  # host-only C++ (no device code): the system compiler
        obj = obj_dir / (Path(src).stem + ".o")
        _run(["g++", *GXX_FLAGS, f"-I{INCLUDE}", "-c", str(CSRC / src), "-o", str(obj)], verbose)
        objs.append(str(obj))
    out = lib_path()
    tmp = out.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-pthread", "-o", str(tmp)], verbose)
    os.replace(tmp, out)
    return out


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}")
    if verbose and (res.stdout or res.stderr):
        sys.stderr.write(res.stdout + res.stderr)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
