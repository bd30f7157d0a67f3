"""The kernels' cos/sin of fp32 angles (chunkkv_amd/csrc/cos_sin.hpp, compiled here for the host
by g++ from the same source): bit-identical to glibc's (float)cos/sin((double)x), the values the
oracle's rotary tables hold (oracle/ckv_oracle.c shift_tables), for EVERY float |x| < 2^31, and
those values correctly rounded (multiprecision spot check). Host code only: no GPU."""

import os
import shutil
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def sweep_bin(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    out = tmp_path_factory.mktemp("cos_sin") / "cos_sin_sweep"
    subprocess.run([gxx, "-O2", "-std=c++17", "-ffp-contract=off", "-pthread", f"-I{ROOT / 'chunkkv_amd' / 'csrc'}",
                    str(ROOT / "tests" / "native" / "cos_sin_sweep.cpp"), "-o", str(out), "-lm"], check=True)
    return out


def _sweep(exe, lo, hi):
    threads = max(1, min(16, os.cpu_count() or 1))
    r = subprocess.run([str(exe), "sweep", str(lo), str(hi), str(threads)], check=True, capture_output=True, text=True)
    lines = r.stdout.split()
    assert lines[-4] == "n" and lines[-2] == "bad", r.stdout
    return int(lines[-3]), int(lines[-1]), r.stdout


def _f32_bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def test_every_float_below_2_pow_31(sweep_bin):
    """All 2 x 0x4f000000 bit patterns: +-0, subnormals, normals up to 2^31 (exclusive)."""
    n, bad, out = _sweep(sweep_bin, 0, _f32_bits(2.0**31))
    assert n == 2 * 0x4F000000
    assert bad == 0, out


def test_out_of_range_angles_are_refused(sweep_bin):
    """2^31 and above, infinities and NaN go to the library sincos (cos_sin_fast returns false)."""
    vals = [2.0**31, -(2.0**31), 3.0e38, float("inf"), float("-inf"), float("nan")]
    inp = "".join(f"{_f32_bits(v):08x}\n" for v in vals)
    r = subprocess.run([str(sweep_bin), "eval"], input=inp, capture_output=True, text=True, check=True)
    assert r.stdout.split() == ["none"] * len(vals)


def test_glibc_values_are_correctly_rounded(sweep_bin):
    """The common target is the correctly rounded fp32 cos/sin: 3000 floats (uniform bit
    patterns below 2^31, plus the rotary angles p * inv_freq at large p) against 200-bit mpmath."""
    mp = pytest.importorskip("mpmath")
    rng = np.random.default_rng(0)
    xs = rng.integers(0, 0x4F000000, 2000, dtype=np.uint32).view(np.float32)
    p = rng.integers(0, 2**31 - 1, 1000)
    inv = (1e6 ** (-(rng.integers(0, 64, 1000) * 2) / 128.0)).astype(np.float32)
    xs = np.concatenate([xs, (p.astype(np.float32) * inv).astype(np.float32)])
    xs = xs[np.abs(xs) < 2.0**31]
    inp = "".join(f"{int(b):08x}\n" for b in xs.view(np.uint32))
    r = subprocess.run([str(sweep_bin), "eval"], input=inp, capture_output=True, text=True, check=True)
    got = [tuple(int(h, 16) for h in line.split()) for line in r.stdout.splitlines()]
    mp.mp.prec = 200
    for x, (cb, sb) in zip(xs, got):
        for fn, b in ((mp.cos, cb), (mp.sin, sb)):
            v = fn(mp.mpf(float(x)))
            d = float(v)  # correctly rounded to fp64; then to fp32 (not at an fp32 midpoint)
            want = np.float32(d)
            lo, hi = np.nextafter(want, np.float32(-np.inf)), np.nextafter(want, np.float32(np.inf))
            assert abs(v - mp.mpf(float(want))) <= min(abs(v - mp.mpf(float(lo))), abs(v - mp.mpf(float(hi))))
            assert int(np.float32(want).view(np.uint32)) == b, (float(x), fn)
