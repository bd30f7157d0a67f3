"""ctypes binding of ``libchunkkv_amd.so`` (declarations: include/chunkkv_amd.h).

torch is imported first so that the library's HIP runtime dependency resolves to the runtime
torch has already loaded: one HIP runtime per process, so torch streams and device pointers are
valid inside the library. There is no fallback: if the library is missing, every op raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libchunkkv_amd.so"
ABI_VERSION = 5

CKV_OK = 0
CKV_ERR_INVALID_ARGUMENT = 1
CKV_ERR_OUT_OF_RANGE = 2
CKV_ERR_TOO_LARGE = 3
CKV_ERR_HIP = 4

DTYPE_F32 = 0
DTYPE_BF16 = 1

COUNT_KEEP = 0
COUNT_SELECTED_CACHED = 1
COUNT_BUDGET = 2
COUNT_CANDIDATES = 3
COUNT_UNCOMPUTED = 4
COUNT_BUDGET_REQUESTED = 5
COUNT_BAD_SPANS = 6
COUNT_TOP_HISTOGRAM = 7  # bit 0: histogram path; bit 1: threshold bin ranked directly
COUNT_N = 8

DEVIATION_SELECT_WORKSPACE_BYTES = 65792
LAYER1_REPAIR_WORKSPACE_BYTES = 65792
POS_POOLED = 8

SELECT_MAX_TOKENS = 131072
DEVICE_ERR_RANGE = 1

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f64 = ctypes.c_double
_f32 = ctypes.c_float

# name -> (restype, argtypes); must match include/chunkkv_amd.h
SIGNATURES = {
    "ckv_abi_version": (_i32, []),
    "ckv_status_string": (ctypes.c_char_p, [_i32]),
    "ckv_inv_freq": (_i32, [_p, _i32, _f64, _p]),
    "ckv_rerope_gather": (
        _i32,
        [_p, _p, _i64, _i64, _p, _i32, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f64, _p, _p],
    ),
    "ckv_rerope_gather_layers": (
        _i32,
        [_p, _p, _i64, _i64, _p, _i32, _i32, _i32, _i32, _p, _i32, _i32, _p, _i32, _i32, _i32, _i32, _f64, _p, _p],
    ),
    "ckv_rerope_gather_layers_kept": (
        _i32,
        [_p, _p, _i64, _i64, _p, _i32, _i32, _i32, _i32, _p, _i32, _i32, _p, _i32, _p, _i64, _i64, _p, _i64, _i64, _p,
         _p, _i32, _p, _i32, _i32, _i32, _i32, _i32, _f64, _p, _p],
    ),
    "ckv_shift_keys": (_i32, [_p, _i64, _p, _i64, _i32, _i32, _i32, _i32, _i32, _f64, _p]),
    "ckv_deviation": (
        _i32,
        [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _i64, _p, _p, _i32, _i32, _i32, _i32, _i32, _p, _p, _p, _p],
    ),
    "ckv_select": (_i32, [_p, _p, _p, _p, _i32, _p, _i32, _i32, _f64, _p, _p, _p, _p, _p, _p, _p]),
    "ckv_assemble_layer": (
        _i32,
        [_p, _p, _i64, _p, _i32, _i32, _i32, _p, _i32, _i32, _p, _i64, _i64, _p, _i64, _i64, _i32, _p, _i32, _i32,
         _i32, _i32, _f64, _p, _p],
    ),
    "ckv_rope_qkv": (
        _i32,
        [_p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _i32, _p, _i64, _i64, _p, _i64, _i64, _p, _i64, _i64,
         _p, _p, _i64, _i32, _i32, _i32, _i32, _i32, _f64, _p, _p],
    ),
    "ckv_rope_table": (_i32, [_p, _i64, _i32, _f64, _p]),
    "ckv_extract_chunks": (
        _i32,
        [_p, _p, _i64, _i64, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _p, _p],
    ),
    "ckv_attention_active": (
        _i32,
        [_p, _p, _i64, _i64, _p, _p, _i64, _p, _i32, _i32, _i32, _i32, _i32, _i32, _f64, _p, _i64, _p, _p],
    ),
    "ckv_attention_workspace_bytes": (_i64, [_i32, _i32, _i32, _i32, _p, _p]),
    "ckv_add_rmsnorm": (_i32, [_p, _p, _p, _p, _p, _i64, _i32, _f32, _i32, _p]),
    "ckv_silu_mul": (_i32, [_p, _i64, _p, _i64, _p, _i64, _i64, _i32, _i32, _p]),
    "ckv_scatter_rows": (
        _i32,
        [_p, _p, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _i32, _i32, _i32, _i32, _i32, _p, _p],
    ),
    "ckv_scatter_kept_rows": (
        _i32,
        [_p, _p, _i64, _p, _i64, _i64, _p, _i64, _i64, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _p, _p],
    ),
    "ckv_deviation_select": (
        _i32,
        [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _i64, _p, _p, _i32, _i32, _i32, _i32, _i32, _p, _i32, _i32, _f64,
         _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _p],
    ),
    "ckv_token_hash_prefixes": (_i32, [_p, _i64, _p, _i32, _p, _i32]),
    "ckv_layer1_repair": (
        _i32,
        [_p, _p, _i64, _p, _i32, _i32, _i32, _p, _i32, _p, _i64, _i64, _p, _i64, _i64, _i32, _p, _p, _i32, _i32, _i32,
         _i32, _f64, _p, _i32, _i32, _f64, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _p],
    ),
    "ckv_layer1_repair_gather": (
        _i32,
        [_p, _p, _i64, _i64, _p, _i32, _i32, _i32, _i32, _i32, _p, _i32, _i32, _p, _i64, _i64, _p, _i64, _i64, _i32,
         _p, _p, _i32, _i32, _i32, _i32, _f64, _p, _i32, _i32, _f64, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p,
         _p],
    ),
    "ckv_layer1_repair_gather_whole_layers": (_i32, [_i32] * 9),
    "ckv_deviation_select_noalloc": (
        _i32,
        [_p, _i64, _i64, _p, _i64, _i64, _p, _p, _i64, _p, _p, _i32, _i32, _i32, _i32, _i32, _p, _i32, _i32, _f64,
         _p, _p, _p, _p, _p, _p, _p, _p, _p, _p],
    ),
}

_lib = None


class NativeLibraryMissing(ImportError):
    pass


def lib() -> ctypes.CDLL:
    """The loaded library; raises NativeLibraryMissing if it was never built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise NativeLibraryMissing(
                f"{LIB_PATH} is not built; run `python -m chunkkv_amd.build` (there is no CPU fallback)"
            )
        handle = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        ver = handle.ckv_abi_version()
        if ver != ABI_VERSION:
            raise NativeLibraryMissing(f"{LIB_PATH} has ABI version {ver}, expected {ABI_VERSION}; rebuild it")
        _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    """Map a ckv_status to the exception the reference path would raise for the same misuse."""
    if status == CKV_OK:
        return
    msg = f"{what}: {lib().ckv_status_string(status).decode()} (status {status})"
    if status in (CKV_ERR_INVALID_ARGUMENT, CKV_ERR_OUT_OF_RANGE, CKV_ERR_TOO_LARGE):
        raise ValueError(msg)
    raise RuntimeError(msg)
