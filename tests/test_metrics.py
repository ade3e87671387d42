"""Known answers for the parity metrics (polykernel_amd/metrics.py).

Mirrors the reference's tests/golden/test_golden_self.py:160-186 (a perfect
match passes with cosine 1, max_rel 0, pcc 1; a +-5 % multiplicative
perturbation must raise) and adds closed-form values of each metric, so a
dropped term, a wrong sign or a swapped operand in a metric fails here.
"""
from __future__ import annotations

import numpy as np
import pytest

from polykernel_amd import metrics
from tests.helpers import bf, f32


def _rand_bf16(n, lo, hi, seed):
    return bf(np.random.default_rng(seed).uniform(lo, hi, size=(n,)))


def test_perfect_match():
    x = _rand_bf16(32, 0.5, 1.5, 0xC0FFEE)
    assert metrics.cosine(x, x) == pytest.approx(1.0, abs=1e-12)
    assert metrics.max_rel_err(x, x) == 0.0
    assert metrics.pcc(x, x) == pytest.approx(1.0, abs=1e-12)
    rep = metrics.assert_correct(x, x)
    assert rep.bit_exact == 1.0 and rep.max_ulp == 0


def test_assert_correct_raises_on_perturbation():
    ref = _rand_bf16(128, 1.0, 2.0, 1)
    noise = np.random.default_rng(1234).uniform(-1.0, 1.0, size=(128,))
    perturbed = bf(f32(ref) * (1.0 + 0.05 * noise))
    assert metrics.max_rel_err(perturbed, ref) > 1e-2
    with pytest.raises(AssertionError, match="assert_correct FAILED"):
        metrics.assert_correct(perturbed, ref)
    # the int8 gate's looser ceiling (quant_golden.py:46-48) accepts 2 % noise
    # that the bf16 gate rejects
    mild = bf(f32(ref) * (1.0 + 0.02 * noise))
    metrics.assert_quant_correct(mild, ref)
    with pytest.raises(AssertionError):
        metrics.assert_correct(mild, ref)


def test_cosine_closed_forms():
    a, b = np.array([1.0, 0.0], np.float32), np.array([0.0, 1.0], np.float32)
    assert metrics.cosine(a, b) == 0.0
    assert metrics.cosine(a, -a) == -1.0
    # cos of [1,2,2] and [2,1,2] = 8/9
    assert metrics.cosine(np.array([1, 2, 2.0]), np.array([2, 1, 2.0])) == pytest.approx(8 / 9, abs=1e-15)
    # scale invariance
    assert metrics.cosine(np.array([3.0, 4.0]), np.array([6.0, 8.0])) == pytest.approx(1.0, abs=1e-15)
    # zero-vector conventions of metrics.py:30-33
    z = np.zeros(3, np.float32)
    assert metrics.cosine(z, z) == 1.0
    assert metrics.cosine(z, np.ones(3, np.float32)) == 0.0


def test_max_rel_err_closed_forms():
    # |a - ref| / (|ref| + 1e-6), maximum over elements; the reference is the denominator
    a = np.array([1.0, 3.0, -2.0], np.float32)
    ref = np.array([1.0, 2.0, -1.0], np.float32)
    assert metrics.max_rel_err(a, ref) == pytest.approx(1.0 / (1.0 + 1e-6), rel=1e-12)
    assert metrics.max_rel_err(ref, a) == pytest.approx(1.0 / (2.0 + 1e-6), rel=1e-12)
    assert metrics.max_rel_err(np.array([1e-6], np.float32), np.array([0.0], np.float32)) == \
        pytest.approx(float(np.float32(1e-6)) / 1e-6, rel=1e-12)


def test_pcc_closed_forms():
    x = np.array([1.0, 2.0, 4.0, 7.0], np.float32)
    assert metrics.pcc(3 * x + 5, x) == pytest.approx(1.0, abs=1e-12)
    assert metrics.pcc(-x, x) == pytest.approx(-1.0, abs=1e-12)
    # [1,2,3] vs [1,3,2]: covariance 0.5*2 / (sqrt(2) sqrt(2)) = 0.5
    assert metrics.pcc(np.array([1, 2, 3.0]), np.array([1, 3, 2.0])) == pytest.approx(0.5, abs=1e-15)
    # zero variance conventions of metrics.py:53-55
    c = np.full(4, 2.0, np.float32)
    assert metrics.pcc(c, c) == 1.0
    assert metrics.pcc(c, c + 1) == 0.0


def test_bf16_inputs_are_decoded_as_bits():
    # uint16 arrays are bf16 codes: 0x3F80 = 1.0, 0x4000 = 2.0, 0xBF80 = -1.0
    a = np.array([0x3F80, 0x4000], np.uint16)
    b = np.array([0x3F80, 0xBF80], np.uint16)
    assert metrics.cosine(a, b) == pytest.approx(-1.0 / np.sqrt(10.0), abs=1e-15)
    assert metrics.max_rel_err(a, b) == pytest.approx(3.0 / (1.0 + 1e-6), rel=1e-12)


def test_ulp_and_bit_exact():
    a = np.array([0x3F80, 0x3F81, 0x0001, 0x8001, 0x0000], np.uint16)
    b = np.array([0x3F80, 0x3F80, 0x8001, 0x0001, 0x8000], np.uint16)
    assert metrics.bit_exact_fraction(a, b) == pytest.approx(1 / 5)
    # +0 and -0 are 0 ulp apart; the smallest subnormals of opposite sign 2 ulp
    assert metrics.max_ulp(a, b) == 2
    assert metrics.max_ulp(np.array([0x7F7F], np.uint16), np.array([0x7F80], np.uint16)) == 1


def test_thresholds_are_the_reference_constants():
    # tests/golden/metrics.py:17-21 and quant_golden.py:46-48
    assert (metrics.COSINE_THRESHOLD, metrics.MAX_REL_ERR_THRESHOLD, metrics.PCC_THRESHOLD,
            metrics.REL_ERR_EPS) == (0.999, 1e-2, 0.99, 1e-6)
    assert (metrics.QUANT_COSINE_THRESHOLD, metrics.QUANT_MAX_REL_ERR_THRESHOLD,
            metrics.QUANT_PCC_THRESHOLD) == (0.99, 5e-2, 0.99)


def test_each_threshold_is_enforced():
    ref = np.linspace(1.0, 2.0, 64)
    rep = metrics.report(bf(ref), bf(ref))
    assert rep.passes()
    # failing only max_rel: one element off by 2 %
    a = ref.copy()
    a[5] *= 1.02
    r = metrics.report(bf(a), bf(ref))
    assert r.cosine >= 0.999 and r.pcc >= 0.99 and not r.passes()
    assert r.passes(rel_t=metrics.LARGE_K_MAX_REL_ERR)
