"""The C-ABI library on a host without a GPU: it loads, exports every entry point declared in
include/chunkkv_amd.h with the ABI version, rejects bad arguments on the host before any launch,
and its structs have the layout the Python side packs. No kernel is launched here."""

import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from chunkkv_amd import _native, ops

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "chunkkv_amd.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int32_t|int64_t|const char\*)\s+(ckv_\w+)\s*\(", text, flags=re.M)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _native.lib()
    names = declared_functions()
    assert len(names) >= 8
    for n in names:
        assert hasattr(lib, n), n
        assert n in _native.SIGNATURES, f"{n} has no ctypes signature"
    assert set(_native.SIGNATURES) == set(names)
    assert lib.ckv_abi_version() == _native.ABI_VERSION
    out = subprocess.run(["nm", "-D", "--defined-only", str(_native.LIB_PATH)], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (ckv_\w+)", out))
    assert set(names) <= exported


def test_status_strings():
    lib = _native.lib()
    assert lib.ckv_status_string(0) == b"ok"
    assert b"invalid" in lib.ckv_status_string(1)
    assert lib.ckv_status_string(99) == b"unknown status"


def test_host_side_argument_validation_never_launches():
    lib = _native.lib()
    # unknown dtype / unsupported head_dim / NULL pointers / bad strides -> errors before any launch
    assert lib.ckv_rerope_gather(1, 1, 10, 10, 1, 1, 1, 1, 1, 1, 1, 1, 128, 7, 1e6, None, None) == _native.CKV_ERR_INVALID_ARGUMENT
    assert lib.ckv_rerope_gather(1, 1, 10, 10, 1, 1, 1, 1, 1, 1, 1, 1, 96, 1, 1e6, None, None) == _native.CKV_ERR_INVALID_ARGUMENT
    assert lib.ckv_rerope_gather(None, 1, 10, 10, 1, 1, 1, 1, 1, 1, 1, 1, 128, 1, 1e6, None, None) == _native.CKV_ERR_INVALID_ARGUMENT
    assert lib.ckv_rerope_gather(1, 1, 100, 10, 1, 1, 1, 1, 1, 1, 1, 1, 128, 1, 1e6, None, None) == _native.CKV_ERR_OUT_OF_RANGE
    assert lib.ckv_rerope_gather(1, 1, 100, 10, 1, 1, 1, 1, 1, 1, 1, 1, 128, 1, -1.0, None, None) == _native.CKV_ERR_INVALID_ARGUMENT
    # layer range: end past n_layers, begin past end -> invalid; empty range -> nothing to do
    assert lib.ckv_rerope_gather_layers(1, 1, 1000, 100, 1, 1, 3, 0, 4, 1, 1, 1, None, 1, 10, 64, 1, 1e6, None, None) \
        == _native.CKV_ERR_INVALID_ARGUMENT
    assert lib.ckv_rerope_gather_layers(1, 1, 1000, 100, 1, 1, 3, 2, 1, 1, 1, 1, None, 1, 10, 64, 1, 1e6, None, None) \
        == _native.CKV_ERR_INVALID_ARGUMENT
    assert lib.ckv_rerope_gather_layers(1, 1, 1000, 640, 1, 1, 3, 2, 2, 1, 1, 1, None, 1, 10, 64, 1, 1e6, None, None) \
        == _native.CKV_OK
    # gather + kept rows: the kept layer inside the gathered range or past n_layers, kept rows with
    # no keep lists, a bad dtype -> invalid; nothing gathered and no kept row -> nothing to do
    kept = lambda *a: lib.ckv_rerope_gather_layers_kept(*a)  # noqa: E731
    kb = [1, 1, 1000, 100, 1, 1, 3, 1, 3, 1, 1, 1, None, 0, 1, 100, 64, 1, 100, 64, 1, 1, 4, None, 10, 1, 10, 64, 1,
          1e6, None, None]
    assert kept(*kb[:13], 2, *kb[14:]) == _native.CKV_ERR_INVALID_ARGUMENT
    assert kept(*kb[:13], 3, *kb[14:]) == _native.CKV_ERR_INVALID_ARGUMENT
    assert kept(*kb[:20], None, *kb[21:]) == _native.CKV_ERR_INVALID_ARGUMENT
    assert kept(*kb[:28], 7, *kb[29:]) == _native.CKV_ERR_INVALID_ARGUMENT
    assert kept(*kb[:2], 1000, 640, *kb[4:7], 2, 2, *kb[9:22], 0, *kb[23:]) == _native.CKV_OK
    assert lib.ckv_inv_freq(None, 128, 1e6, None) == _native.CKV_ERR_INVALID_ARGUMENT
    assert lib.ckv_inv_freq(1, 127, 1e6, None) == _native.CKV_ERR_INVALID_ARGUMENT
    assert lib.ckv_shift_keys(1, 10, 1, 10, 1, 1, 100, 1, 3, 1e6, None) == _native.CKV_ERR_INVALID_ARGUMENT
    assert lib.ckv_deviation(1, 1, 1, 1, 1, 1, 1, 1, 512, 1, 1, 4, 4, 4, 128, 5, 1, 1, None, None) == _native.CKV_ERR_INVALID_ARGUMENT
    assert lib.ckv_deviation(1, 1, 1, 1, 1, 1, 1, 1, 10, 1, 1, 4, 4, 4, 128, 1, 1, 1, None, None) == _native.CKV_ERR_OUT_OF_RANGE
    assert lib.ckv_select(1, 1, 1, 1, _native.SELECT_MAX_TOKENS + 1, 1, 1, 0, 0.0, 1, 1, None, 1, 1, 1, None) == _native.CKV_ERR_TOO_LARGE
    assert lib.ckv_select(None, 1, 1, 1, 10, 1, 1, 0, 0.0, 1, 1, None, 1, 1, 1, None) == _native.CKV_ERR_INVALID_ARGUMENT
    # assemble: bad dtype, layer outside [0, n_layers), short head stride, fresh rows missing
    asm = lambda *a: lib.ckv_assemble_layer(*a)  # noqa: E731
    base = [1, 1, 1024, 1, 1, 2, 0, 1, 1, 8, 1, 128, 128, 1, 128, 128, 8, 1, 8, 1, 128, 1, 1e6, None, None]
    assert asm(*base[:21], 9, *base[22:]) == _native.CKV_ERR_INVALID_ARGUMENT
    assert asm(*base[:6], 2, *base[7:]) == _native.CKV_ERR_INVALID_ARGUMENT
    assert asm(*base[:2], 10, *base[3:]) == _native.CKV_ERR_OUT_OF_RANGE
    assert asm(*base[:10], None, *base[11:]) == _native.CKV_ERR_INVALID_ARGUMENT
    assert asm(*base[:7], 1, 0, *base[9:]) == _native.CKV_OK  # no segments: nothing to do
    assert lib.ckv_scatter_rows(1, 1, 10, 1, 1, 1, 1, 1, 1, 1, 4, 10, 4, 128, 1, None, None) == _native.CKV_ERR_OUT_OF_RANGE
    assert lib.ckv_scatter_rows(1, 1, 10, 1, 1, 1, 1, 1, 1, 1, 4, 10, 4, 100, 1, None, None) == _native.CKV_ERR_INVALID_ARGUMENT
    # zero-sized work is a no-op success
    assert lib.ckv_scatter_rows(None, None, 0, None, 0, 0, None, 0, 0, None, 0, 0, 4, 128, 1, None, None) == _native.CKV_OK


def test_status_maps_to_reference_exception_types():
    with pytest.raises(ValueError):
        _native.check(_native.CKV_ERR_INVALID_ARGUMENT, "x")
    with pytest.raises(ValueError):
        _native.check(_native.CKV_ERR_TOO_LARGE, "x")
    with pytest.raises(RuntimeError):
        _native.check(_native.CKV_ERR_HIP, "x")
    _native.check(_native.CKV_OK, "x")


def test_ops_refuse_host_tensors():
    k = torch.zeros(1, 2, 4, 64)
    with pytest.raises(ValueError, match="HIP device"):
        ops.shift_keys(k, 3, 1e6)
    with pytest.raises(ValueError, match="HIP device"):
        ops.scatter_rows(k, k, k, k, torch.zeros(4, dtype=torch.int64))
    with pytest.raises(TypeError):
        ops.dtype_code(torch.float16)
    assert ops.shift_keys(k, 0, 1e6) is k  # delta 0 returns the input before any device check


def test_engine_refuses_cpu_model():
    from chunkkv_amd.engine import HipEngine
    from tests.helpers import StubTokenizer, tiny_qwen2

    with pytest.raises(ValueError, match="HIP device"):
        HipEngine(tiny_qwen2(layers=1, hidden=64, heads=1, kv=1, inter=64, vocab=32), StubTokenizer())


def test_struct_layouts_match_header(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "chunkkv_amd.h"\n'
        "int main(void){printf(\"%zu %zu %zu %zu %zu %d %d %d\\n\", sizeof(ckv_segment), offsetof(ckv_segment, delta),"
        " sizeof(ckv_chunk_span), offsetof(ckv_chunk_span, pooled), offsetof(ckv_segment, src_len),"
        " CKV_COUNT_N, CKV_SELECT_MAX_TOKENS, CKV_ABI_VERSION); return 0;}\n"
    )
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    vals = list(map(int, subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()))
    assert vals == [24, 20, 16, 12, 16, _native.COUNT_N, _native.SELECT_MAX_TOKENS, _native.ABI_VERSION]
    from chunkkv_amd.planner import SEG_FIELDS, SPAN_FIELDS

    assert SEG_FIELDS * 4 == 24 and SPAN_FIELDS * 4 == 16
    assert np.dtype(np.int32).itemsize == 4
    assert ctypes.sizeof(ctypes.c_void_p) == 8


def test_attention_workspace_sizing_is_host_only():
    """The split decision for the attention: decode-like shapes split, big launches do not."""
    lib = _native.lib()
    s, t = ctypes.c_int32(0), ctypes.c_int32(0)
    nb = lib.ckv_attention_workspace_bytes(1, 8256, 28, 128, ctypes.byref(s), ctypes.byref(t))
    row = 28 * 1 * 132 * 4  # one partial row per query head: D fp32 + (max, sum) + pad
    # sized for the larger of the per-head split plan and the grouped plan (3-tile splits: 43)
    assert s.value > 1 and t.value * s.value >= (8256 + 63) // 64 and nb == max(s.value, 43) * row
    assert lib.ckv_attention_workspace_bytes(2976, 8256, 28, 128, None, None) == 0
    assert lib.ckv_attention_workspace_bytes(1, 100, 28, 128, None, None) == 0  # short cache: no split


def test_norm_and_gate_validation_never_launches():
    lib = _native.lib()
    bf16, f32 = 1, 0
    norm = lambda *a: lib.ckv_add_rmsnorm(*a)  # noqa: E731
    assert norm(1, 1, 1, 1, 1, 4, 8200, 1e-6, bf16, None) == _native.CKV_ERR_TOO_LARGE  # > 8192 elements
    assert norm(1, 1, 1, 1, 1, 4, 4100, 1e-6, f32, None) == _native.CKV_ERR_TOO_LARGE  # > 4096 fp32
    assert norm(1, 1, 1, 1, 1, 4, 100, 1e-6, bf16, None) == _native.CKV_ERR_INVALID_ARGUMENT  # not a multiple of 8
    assert norm(1, 1, 1, 1, 1, 4, 128, 1e-6, 7, None) == _native.CKV_ERR_INVALID_ARGUMENT  # dtype
    assert norm(None, 1, 1, 1, 1, 4, 128, 1e-6, bf16, None) == _native.CKV_ERR_INVALID_ARGUMENT  # add needs h_out
    assert norm(1, 1, 1, 1, 1, 4, 128, -1.0, bf16, None) == _native.CKV_ERR_INVALID_ARGUMENT
    assert norm(1, 1, 1, 1, 1, -1, 128, 1e-6, bf16, None) == _native.CKV_ERR_INVALID_ARGUMENT
    assert norm(None, None, None, None, None, 0, 128, 1e-6, bf16, None) == _native.CKV_OK  # no rows
    gate = lambda *a: lib.ckv_silu_mul(*a)  # noqa: E731
    assert gate(1, 64, 1, 32, 1, 64, 4, 64, bf16, None) == _native.CKV_ERR_OUT_OF_RANGE  # row stride < width
    assert gate(1, 64, 1, 68, 1, 64, 4, 64, bf16, None) == _native.CKV_ERR_INVALID_ARGUMENT  # unaligned stride
    assert gate(1, 60, 1, 60, 1, 60, 4, 60, bf16, None) == _native.CKV_ERR_INVALID_ARGUMENT  # width % 8
    assert gate(None, 64, 1, 64, 1, 64, 4, 64, bf16, None) == _native.CKV_ERR_INVALID_ARGUMENT
    assert gate(None, 64, None, 64, None, 64, 0, 64, bf16, None) == _native.CKV_OK
