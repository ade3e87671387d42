"""Parity metrics and the correctness gate.

Definitions follow the reference's tests/golden/metrics.py:20-77 (flattened,
fp32-upcast view; cosine, max relative error with eps 1e-6, Pearson
correlation) and its thresholds (cosine >= 0.999, max_rel <= 1e-2,
pcc >= 0.99); the int8 gate uses tests/golden/quant_golden.py:46-48
(0.99 / 5e-2 / 0.99).  All sums are taken in float64.  Besides the three
metrics a report carries the bit-exact fraction and the maximum distance in
bf16 units in the last place (ulp).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

COSINE_THRESHOLD = 0.999
MAX_REL_ERR_THRESHOLD = 1e-2
PCC_THRESHOLD = 0.99
REL_ERR_EPS = 1e-6
QUANT_COSINE_THRESHOLD = 0.99
QUANT_MAX_REL_ERR_THRESHOLD = 5e-2
QUANT_PCC_THRESHOLD = 0.99
# The reference's own calibrated ceiling for long fp32 reductions
# (tests/kernels/test_hip_run.py:80, lib/Autotune/Benchmark.h:88-91).
LARGE_K_MAX_REL_ERR = 5e-2


def _f(x) -> np.ndarray:
    x = np.asarray(x)
    if x.dtype == np.uint16:  # bf16 bits
        x = (x.astype(np.uint32) << 16).view(np.float32)
    return x.astype(np.float64).reshape(-1)


def cosine(a, ref) -> float:
    x, y = _f(a), _f(ref)
    nx, ny = np.linalg.norm(x), np.linalg.norm(y)
    if nx * ny == 0.0:
        return 1.0 if (nx == 0.0 and ny == 0.0) else 0.0
    return float(np.dot(x, y) / (nx * ny))


def max_rel_err(a, ref, eps: float = REL_ERR_EPS) -> float:
    x, y = _f(a), _f(ref)
    if x.size == 0:
        return 0.0
    return float(np.max(np.abs(x - y) / (np.abs(y) + eps)))


def pcc(a, ref) -> float:
    x, y = _f(a), _f(ref)
    xc, yc = x - x.mean(), y - y.mean()
    den = np.sqrt(np.sum(xc * xc)) * np.sqrt(np.sum(yc * yc))
    if den == 0.0:
        return 1.0 if np.array_equal(x, y) else 0.0
    return float(np.sum(xc * yc) / den)


def _ordered(b: np.ndarray) -> np.ndarray:
    """Map bf16 bits onto a monotone integer line (for ulp distances)."""
    v = b.astype(np.int64)
    return np.where(v & 0x8000, -(v & 0x7FFF), v & 0x7FFF)


def bit_exact_fraction(a_bits: np.ndarray, ref_bits: np.ndarray) -> float:
    a, r = np.asarray(a_bits).reshape(-1), np.asarray(ref_bits).reshape(-1)
    return float(np.mean(a == r)) if a.size else 1.0


def max_ulp(a_bits: np.ndarray, ref_bits: np.ndarray) -> int:
    a, r = np.asarray(a_bits).reshape(-1), np.asarray(ref_bits).reshape(-1)
    if a.size == 0:
        return 0
    return int(np.max(np.abs(_ordered(a) - _ordered(r))))


@dataclass
class Report:
    cosine: float
    max_rel_err: float
    pcc: float
    bit_exact: float
    max_ulp: int

    def passes(self, cos_t=COSINE_THRESHOLD, rel_t=MAX_REL_ERR_THRESHOLD, pcc_t=PCC_THRESHOLD) -> bool:
        return self.cosine >= cos_t and self.max_rel_err <= rel_t and self.pcc >= pcc_t

    def __str__(self) -> str:
        return (f"cosine={self.cosine:.7f} max_rel_err={self.max_rel_err:.3e} pcc={self.pcc:.7f} "
                f"bit_exact={self.bit_exact:.6f} max_ulp={self.max_ulp}")


def report(a_bits, ref_bits) -> Report:
    """Metrics of bf16 outputs given as uint16 bit arrays."""
    a, r = np.asarray(a_bits, dtype=np.uint16), np.asarray(ref_bits, dtype=np.uint16)
    return Report(cosine(a, r), max_rel_err(a, r), pcc(a, r), bit_exact_fraction(a, r), max_ulp(a, r))


def assert_correct(a_bits, ref_bits, rel_t: float = MAX_REL_ERR_THRESHOLD, what: str = "") -> Report:
    rep = report(a_bits, ref_bits)
    if not rep.passes(rel_t=rel_t):
        raise AssertionError(f"{what} assert_correct FAILED: {rep} (rel ceiling {rel_t:g})")
    return rep


def assert_quant_correct(a_bits, ref_bits, what: str = "") -> Report:
    rep = report(a_bits, ref_bits)
    if not rep.passes(QUANT_COSINE_THRESHOLD, QUANT_MAX_REL_ERR_THRESHOLD, QUANT_PCC_THRESHOLD):
        raise AssertionError(f"{what} assert_quant_correct FAILED: {rep}")
    return rep
