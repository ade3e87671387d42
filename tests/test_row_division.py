"""The row kernels divide by the row's RMS with a three-operation exact method
(rowwise.hip div_fast: reciprocal, product, one fma correction) instead of the
IEEE division sequence.  It must give the division's bits for every input the
kernels send down that path.

CPU: tests/cpp/row_division_check.c, compiled with gcc -ffp-contract=off,
compares the method with IEEE x / d for all 65536 bf16 numerators x 2000
divisors.  GPU: pk_check_row_division compares the device implementation
with the device's own IEEE division over every bf16 numerator for 4096
divisors.  A method that skipped the correction step (q = x * RN(1/d)) fails
both: the CPU check plants that mistake and expects mismatches.  The packed
range test that picks the fast path (DivSpan: two bf16 magnitudes per word,
packed 16-bit min / max) is checked against the float test for every code,
on the CPU (with a planted off-by-one bound that must fail) and on the device.
"""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
SRC = ROOT / "tests" / "cpp" / "row_division_check.c"


def _build(tmp_path, extra=()):
    cc = shutil.which("gcc")
    if cc is None:
        pytest.skip("no gcc")
    exe = tmp_path / "row_division_check"
    r = subprocess.run([cc, "-O2", "-ffp-contract=off", "-fno-fast-math", *extra, str(SRC), "-o", str(exe), "-lm"],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def _summary(r):
    """The division sweep's closing line: "checked N, fast path F, mismatches M"."""
    return r.stdout.strip().splitlines()[-1]


def test_division_method_matches_ieee_on_cpu(tmp_path):
    exe = _build(tmp_path)
    r = subprocess.run([str(exe), "2000"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and _summary(r).endswith("mismatches 0") and "span mismatches 0" in r.stdout, r.stdout


def test_check_detects_a_missing_correction(tmp_path):
    """The same check with the correction step removed must report mismatches
    (the check can fail)."""
    exe = _build(tmp_path, ["-DPK_PLANT_NO_CORRECTION"])
    r = subprocess.run([str(exe), "200"], capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and not _summary(r).endswith("mismatches 0"), r.stdout


def test_check_detects_a_wrong_range_bound(tmp_path):
    """The packed range test with its upper bound off by one (2^64 accepted)
    must report mismatches."""
    exe = _build(tmp_path, ["-DPK_PLANT_SPAN_BOUND"])
    r = subprocess.run([str(exe), "1"], capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and "span mismatches 0" not in r.stdout, r.stdout


@pytest.mark.gpu
def test_device_division_matches_ieee(gpu):
    import ctypes

    from polykernel_amd import _lib

    rng = np.random.default_rng(0x0D17)
    mant = rng.integers(0, 1 << 23, size=4000, dtype=np.uint32)
    expo = rng.integers(127 - 30, 127 + 30, size=4000, dtype=np.uint32)
    ds = ((expo << 23) | mant).view(np.float32)
    edges = np.array([2.0**-30, 2.0**30, np.nextafter(np.float32(2.0**30), np.float32(0)), 1.0, 1e-3, 0.5,
                      np.sqrt(np.float32(1e-6)), 1.0000001, 1.9999999, 3.0], np.float32)
    ds = np.ascontiguousarray(np.concatenate([edges, ds[: 4096 - edges.size]]).astype(np.float32))
    bad = ctypes.c_ulonglong(123)
    _lib.check(_lib.load().pk_check_row_division(ds.ctypes.data, ds.size, ctypes.byref(bad)), "row division")
    assert bad.value == 0
