"""GPU parity: every entry point through the C-ABI against the C oracle.

Bars (written per test):
  * bit-exact: GELU (all 65536 codes), KV append, int8 quantisation, GEMMs on
    integer-valued inputs (exact sums in any order);
  * reference thresholds (cosine >= 0.999, PCC >= 0.99, max rel err <= 1e-2,
    tests/golden/metrics.py:19-23) for rmsnorm / softmax / elementwise-exact
    epilogues, plus a bit-exact fraction floor;
  * for long fp32 reductions (GEMMs, attention) max rel err <= 1e-2 cannot hold
    at outputs that are ~0 relative to their terms (the reference hit this
    itself: tests/kernels/test_hip_run.py:24-31, reports/w5_bench.log:22-27), so
    besides cosine/PCC and a bit-exact floor each element must satisfy an
    explicit fp32 error model, e.g. |gpu - oracle| <= 2 bf16 ulp(|oracle|)
    + K 2^-23 sum_k |a_k b_k| for a GEMM -- true for any fp32 summation order,
    false for a wrong index, sign or dropped term.
"""
from __future__ import annotations

import numpy as np
import pytest

from polykernel_amd import metrics as mt
from polykernel_amd import synth
from tests.bounds import _abs_dot, _att_bound_bad, _err_bound_ok, _gate_bad, _gate_int8_bad, _int8_exact_inputs
from tests.helpers import bf, f32, from_dev, int_bf16, rng_bf16, to_dev

pytestmark = pytest.mark.gpu


def K():
    from polykernel_amd import kernels

    return kernels


def _say(msg):
    print(msg, flush=True)


# ------------------------------------------------------------------ elementwise / rows

def test_device_bf16_conversion_exhaustive(gpu):
    """All 2^32 fp32 inputs: the kernels' hardware fp32->bf16 conversion equals
    the reference RNE formula (kernels/cpu/cpu_reference.h:52-61)."""
    import ctypes
    from polykernel_amd import _lib

    bad = ctypes.c_ulonglong(123)
    _lib.check(_lib.load().pk_check_bf16_conversion(ctypes.byref(bad)), "pk_check_bf16_conversion")
    assert bad.value == 0


def test_paired_gelu_equals_exact_gelu(gpu):
    """The GEMM epilogue's two-codes-per-register GELU equals the per-element
    exact GELU for every code in the low half (x four high-half patterns), on
    its common path and through its NaN/infinity fallback."""
    import ctypes
    from polykernel_amd import _lib

    bad = ctypes.c_ulonglong(123)
    _lib.check(_lib.load().pk_check_gelu_pairs(ctypes.byref(bad)), "pk_check_gelu_pairs")
    assert bad.value == 0


def test_gelu_all_bf16_codes_bit_exact(gpu, oracle):
    x = np.arange(1 << 16, dtype=np.uint16)
    got = from_dev(K().gelu(to_dev(x)))
    want = oracle.gelu(x)
    nan = ((x & 0x7F80) == 0x7F80) & ((x & 0x7F) != 0)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all(((got[nan] & 0x7F80) == 0x7F80) & ((got[nan] & 0x7F) != 0))


@pytest.mark.parametrize("rows,cols,gamma", [(2048, 4096, False), (128, 768, True), (7, 130, True),
                                             (64, 8192, True), (3, 16384, False), (5, 24, False),
                                             (4, 20000, True), (3, 65536, False), (2, 131072, True)])
def test_rmsnorm(gpu, oracle, rows, cols, gamma):
    _say(f"rmsnorm {rows}x{cols} gamma={gamma}")
    x = synth.normal_bf16((rows, cols), 1)
    g = synth.normal_bf16((cols,), 2, 0.1, 1.0) if gamma else None
    got = from_dev(K().rmsnorm(to_dev(x), None if g is None else to_dev(g), 1e-6))
    want = oracle.rmsnorm(x, g, 1e-6)
    rep = mt.assert_correct(got, want, what="rmsnorm")
    assert rep.bit_exact >= 0.99 and rep.max_ulp <= 1, rep


@pytest.mark.parametrize("rows,cols", [(256, 8192), (31, 1000), (16384, 8192)])
def test_residual_rmsnorm(gpu, oracle, rows, cols):
    _say(f"residual_rmsnorm {rows}x{cols}")
    x, r = synth.normal_bf16((rows, cols), 3), synth.normal_bf16((rows, cols), 4)
    g = synth.normal_bf16((cols,), 5, 0.1, 1.0)
    got = from_dev(K().fused_residual_rmsnorm(to_dev(x), to_dev(r), to_dev(g), 1e-6))
    want = oracle.residual_rmsnorm(x, r, g, 1e-6)
    rep = mt.assert_correct(got, want, what="residual_rmsnorm")
    assert rep.bit_exact >= 0.99 and rep.max_ulp <= 1, rep


@pytest.mark.parametrize("rows,cols", [(8, 16), (64, 1000), (128, 8192), (3, 2), (2, 20000), (3, 65536),
                                       (2, 131072)])
def test_softmax(gpu, oracle, rows, cols):
    _say(f"softmax {rows}x{cols}")
    x = rng_bf16((rows, cols), 6, -8, 8)
    got = from_dev(K().softmax(to_dev(x)))
    want = oracle.softmax(x)
    rep = mt.assert_correct(got, want, what="softmax")
    assert rep.bit_exact >= 0.98, rep


def test_softmax_known_uniform(gpu):
    got = f32(from_dev(K().softmax(to_dev(bf([[1.0, 1.0]])))))
    assert np.array_equal(got, np.array([[0.5, 0.5]], np.float32))


@pytest.mark.parametrize("rows,cols", [(64, 8192), (33, 777), (16384, 8192)])
def test_softmax_mask(gpu, oracle, rows, cols):
    _say(f"softmax_mask {rows}x{cols}")
    logits = synth.normal_f32((rows, cols), 7, 2.0)
    mask = synth.mask_bf16((rows, cols), 8, 0.1)
    got = from_dev(K().fused_softmax_mask(to_dev(logits), to_dev(mask)))
    want = oracle.softmax_mask(logits, mask)
    rep = mt.assert_correct(got, want, what="softmax_mask")
    assert rep.bit_exact >= 0.98, rep
    assert np.all(f32(got)[mask == 0xFF80] == 0.0)


@pytest.mark.parametrize("rows,cols", [(37, 2048), (37, 4096), (37, 6000), (37, 8192), (21, 12000), (37, 16384),
                                       (13, 32768), (5, 40000), (7, 65536), (3, 70000), (3, 128256), (2, 131072),
                                       (2, 140000)])
def test_row_ops_every_config(gpu, oracle, rows, cols):
    """Every candidate of residual + RMSNorm and masked softmax (one wave per
    row, a workgroup of 4, 8 or 16 waves per row, the packed-bf16 kernel up to
    131072 columns, the generic kernel past them; ragged rows and widths that
    leave lanes idle) through pk_*_config against the oracle."""
    from polykernel_amd import runtime as rt

    x, r = synth.normal_bf16((rows, cols), 3), synth.normal_bf16((rows, cols), 4)
    g = synth.normal_bf16((cols,), 5, 0.1, 1.0)
    logits, mask = synth.normal_f32((rows, cols), 7, 2.0), synth.mask_bf16((rows, cols), 8, 0.1)
    want_r = oracle.residual_rmsnorm(x, r, g, 1e-6)
    want_s = oracle.softmax_mask(logits, mask)
    for op in ("fused_residual_rmsnorm", "fused_softmax_mask"):
        cands = rt.candidates(op, rows, cols, 0)
        assert cands and cands[0] == rt.default_config(op, rows, cols, 0)
        for cfg in cands:
            _say(f"{op} {rows}x{cols} {cfg}")
            if op == "fused_residual_rmsnorm":
                got = from_dev(K().fused_residual_rmsnorm(to_dev(x), to_dev(r), to_dev(g), 1e-6, config=cfg))
                rep = mt.assert_correct(got, want_r, what=op)
                assert rep.bit_exact >= 0.99 and rep.max_ulp <= 1, (cfg, rep)
            else:
                got = from_dev(K().fused_softmax_mask(to_dev(logits), to_dev(mask), config=cfg))
                rep = mt.assert_correct(got, want_s, what=op)
                assert rep.bit_exact >= 0.98, (cfg, rep)
                assert np.all(f32(got)[mask == 0xFF80] == 0.0)


@pytest.mark.parametrize("cols", [98304, 131072])
def test_softmax_mask_rising_max_rows(gpu, oracle, cols):
    """Rows of 65537-131072 columns take the packed-bf16 softmax, which sums
    online: each lane's running sum is rescaled by exp(m_old - m_new) whenever
    its running max grows, so the sum differs from the oracle's two-pass
    sum of exp(z - m) in the last fp32 bits.  Rows whose max keeps rising (a
    gentle and a steep ramp under noise: the max grows on nearly every chunk
    a lane reads), one whose max falls and an ordinary one exercise that
    rescaling against the row bars (>= 98 % bit-exact, <= 1 ulp)."""
    rows = 4
    c = np.arange(cols, dtype=np.float32)
    logits = synth.normal_f32((rows, cols), 91, 1.0)
    logits[0] += c * np.float32(30.0 / cols)
    logits[1] += c * np.float32(200.0 / cols)
    logits[2] -= c * np.float32(30.0 / cols)
    mask = synth.mask_bf16((rows, cols), 92, 0.1)
    _say(f"softmax rising max {cols}")
    got = from_dev(K().fused_softmax_mask(to_dev(logits), to_dev(mask)))
    want = oracle.softmax_mask(logits, mask)
    rep = mt.assert_correct(got, want, what="softmax_mask rising max")
    assert rep.bit_exact >= 0.98 and rep.max_ulp <= 1, rep
    assert np.all(f32(got)[mask == 0xFF80] == 0.0)


@pytest.mark.parametrize("cols", [1000, 8192, 65536, 131072])
def test_softmax_mask_special_rows(gpu, oracle, cols):
    """Rows the online and two-pass sums must treat as the oracle does, on every
    config: all positions masked (max -inf: NaN everywhere), one position
    unmasked (exactly 1 there, 0 elsewhere), a +inf logit (NaN everywhere), the
    +inf in the last chunk after finite values, and an ordinary row."""
    from polykernel_amd import runtime as rt

    rows = 5
    logits = synth.normal_f32((rows, cols), 21, 2.0)
    mask = synth.mask_bf16((rows, cols), 22, 0.1)
    mask[0, :] = 0xFF80
    mask[1, :] = 0xFF80
    mask[1, cols // 3] = 0
    logits[2, 7] = np.inf
    logits[3, cols - 1] = np.inf
    want = oracle.softmax_mask(logits, mask)
    wf = f32(want)
    assert np.all(np.isnan(wf[[0, 2, 3]])) and wf[1, cols // 3] == 1.0
    for cfg in rt.candidates("fused_softmax_mask", rows, cols, 0):
        _say(f"softmax special rows {cols} {cfg}")
        got = f32(from_dev(K().fused_softmax_mask(to_dev(logits), to_dev(mask), config=cfg)))
        assert np.array_equal(np.isnan(got), np.isnan(wf)), cfg
        assert np.array_equal(got[1], wf[1]), cfg
        rep = mt.report(from_dev(K().fused_softmax_mask(to_dev(logits[4:]), to_dev(mask[4:]), config=cfg)),
                        want[4:])
        assert rep.cosine >= 0.999 and rep.bit_exact >= 0.98, (cfg, rep)


def test_row_config_refusals(gpu):
    """A config outside the shape's list is an argument error; a vector config
    with operands that are not 16-byte aligned is refused (the built-in choice
    then takes the generic kernel)."""
    import torch
    from polykernel_amd import _lib
    from polykernel_amd import runtime as rt

    lib = _lib.load()
    rows, cols = 8, 8192
    xs = torch.zeros(rows * cols + 8, dtype=torch.bfloat16, device="cuda")
    out = torch.zeros(rows * cols + 8, dtype=torch.bfloat16, device="cuda")
    ptr = xs.data_ptr()
    wrong = _lib.Config(4, cols, 0, 4, 8, 1, 1)  # one wave per row cannot hold 1024 vectors
    rc = lib.pk_fused_residual_rmsnorm_config(ptr, ptr, None, out.data_ptr(), rows, cols, 1e-6, wrong, None)
    assert rc == _lib.PK_ERR_INVALID_ARG and "is not a row config" in _lib.last_error()
    cfg = _lib.Config(**rt.default_config("fused_residual_rmsnorm", rows, cols, 0))
    rc = lib.pk_fused_residual_rmsnorm_config(ptr + 2, ptr + 2, None, out.data_ptr() + 2, rows, cols, 1e-6, cfg, None)
    assert rc == _lib.PK_ERR_UNSUPPORTED and "16-byte aligned" in _lib.last_error()
    logits = torch.zeros(rows * cols + 4, dtype=torch.float32, device="cuda")
    cfg = _lib.Config(**rt.default_config("fused_softmax_mask", rows, cols, 0))
    rc = lib.pk_fused_softmax_mask_config(logits.data_ptr() + 4, ptr, out.data_ptr(), rows, cols, cfg, None)
    assert rc == _lib.PK_ERR_UNSUPPORTED and "16-byte aligned" in _lib.last_error()
    torch.cuda.synchronize()


def test_kv_cache_update_bit_exact(gpu, oracle):
    cache, new = rng_bf16((1, 4, 100, 128), 9), rng_bf16((1, 4, 28, 128), 10)
    got = from_dev(K().kv_cache_update(to_dev(cache), to_dev(new)))
    assert np.array_equal(got, oracle.kv_append(cache, new))
    cache, new = rng_bf16((2, 3, 8, 40), 11), rng_bf16((2, 3, 5, 40), 12)
    got = from_dev(K().kv_cache_update(to_dev(cache), to_dev(new)))
    assert np.array_equal(got, oracle.kv_append(cache, new))


@pytest.mark.parametrize("Kd,N", [(128, 128), (130, 127), (8192, 2048), (7, 3)])
def test_quantize_bit_exact(gpu, oracle, Kd, N):
    w = synth.normal_bf16((Kd, N), 13, 1.0 / np.sqrt(Kd))
    w[:, 0] = 0
    wq, s = K().quantize_per_channel(to_dev(w))
    owq, os_ = oracle.quantize_per_channel(w)
    assert np.array_equal(from_dev(s).view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(from_dev(wq), owq)


def test_quantize_rows_beyond_one_grid_pass(gpu, oracle):
    """K above 65535 x 128 rows: the amax kernel's row chunks wrap around the
    grid's y extent; a column whose largest magnitude sits only in the last
    rows checks that those rows are reached."""
    Kd, N = 65535 * 128 + 384, 8
    _say(f"quantize K={Kd} N={N}")
    w = synth.normal_bf16((Kd, N), 16, 1.0 / np.sqrt(Kd))
    w[-1, 1] = bf([3.0])[0]
    w[-200, 2] = bf([-5.0])[0]
    wq, s = K().quantize_per_channel(to_dev(w))
    owq, os_ = oracle.quantize_per_channel(w)
    assert np.array_equal(from_dev(s).view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(from_dev(wq), owq)
    assert from_dev(wq)[-1, 1] == 127 and from_dev(wq)[-200, 2] == -127


def test_quantize_ties_bit_exact(gpu, oracle):
    col = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5], np.float32)
    w = bf(np.tile(col[:, None], (1, 16)))
    wq, s = K().quantize_per_channel(to_dev(w))
    assert list(from_dev(wq)[:, 0]) == [127, 0, 2, 2, 0, -2, -2, 126]


# ------------------------------------------------------------------ GEMM family

@pytest.mark.parametrize("tile", [0, 1, 2, 3])
@pytest.mark.parametrize("M,N,Kd", [(256, 256, 512), (130, 65, 127), (300, 520, 200), (300, 520, 224),
                                    (513, 264, 32), (1024, 768, 1056)])
def test_gemm_integer_inputs_bit_exact(gpu, oracle, tile, M, N, Kd):
    _say(f"gemm int tile={tile} {M}x{N}x{Kd}")
    a, b = int_bf16((M, Kd), 14), int_bf16((Kd, N), 15)
    got = from_dev(K().gemm_ex(0, to_dev(a), to_dev(b), tile=tile))
    assert np.array_equal(got, oracle.matmul(a, b))


@pytest.mark.parametrize("tile", [-1, 0, 1, 2, 3])
@pytest.mark.parametrize("M,N,Kd", [(1, 1, 1), (1, 8, 32), (3, 7, 5), (2, 264, 64), (257, 9, 96)])
def test_gemm_tiny_shapes_bit_exact(gpu, oracle, tile, M, N, Kd):
    """Degenerate but valid shapes (a single row, column or k, tiles mostly
    outside the matrix) on every tile choice, integer inputs: bit-exact."""
    _say(f"gemm tiny tile={tile} {M}x{N}x{Kd}")
    a, b = int_bf16((M, Kd), 16), int_bf16((Kd, N), 17)
    got = from_dev(K().gemm_ex(0, to_dev(a), to_dev(b), tile=tile))
    assert np.array_equal(got, oracle.matmul(a, b)), (tile, M, N, Kd)


def test_matmul_known_2x2(gpu):
    got = f32(from_dev(K().matmul(to_dev(bf([[1, 2], [3, 4]])), to_dev(bf([[5, 6], [7, 8]])))))
    assert np.array_equal(got, np.array([[19, 22], [43, 50]], np.float32))


@pytest.mark.parametrize("M,N,Kd", [(128, 3072, 768), (130, 65, 127), (512, 1024, 4096), (64, 64, 64),
                                    (1024, 2048, 2048)])
def test_matmul_random(gpu, oracle, M, N, Kd):
    _say(f"matmul {M}x{N}x{Kd}")
    a = synth.normal_bf16((M, Kd), 16)
    b = synth.normal_bf16((Kd, N), 17, 1.0 / np.sqrt(Kd))
    got = from_dev(K().matmul(to_dev(a), to_dev(b)))
    want = oracle.matmul(a, b)
    rep = mt.report(got, want)
    assert rep.passes(rel_t=mt.LARGE_K_MAX_REL_ERR if Kd >= 256 else mt.MAX_REL_ERR_THRESHOLD) or \
        (rep.cosine >= 0.999 and rep.pcc >= 0.99), rep
    assert _err_bound_ok(got, want, _abs_dot(a, b), Kd) == 0, rep


@pytest.mark.parametrize("M,N,Kd", [(130, 200, 832), (33, 72, 128), (64, 3072, 768)])
def test_fused_rmsnorm_matmul_gamma_shapes(gpu, oracle, M, N, Kd):
    x = synth.normal_bf16((M, Kd), 26)
    g = synth.normal_bf16((Kd,), 27, 0.1, 1.0)
    w = synth.normal_bf16((Kd, N), 28, 1.0 / np.sqrt(Kd))
    got = from_dev(K().fused_rmsnorm_matmul(to_dev(x), to_dev(w), to_dev(g), 1e-6))
    want = oracle.fused_rmsnorm_matmul(x, w, g, 1e-6)
    rep = mt.report(got, want)
    assert rep.cosine >= 0.999 and rep.pcc >= 0.99 and rep.bit_exact >= 0.98, rep
    a = oracle.rmsnorm(x, g, 1e-6)
    assert _err_bound_ok(got, want, _abs_dot(a, w), Kd, operand_ulps=1.0) == 0, rep


def test_fused_rmsnorm_matmul_config1(gpu, oracle):
    """Config 1: x [128,768] N(0,1), gamma 1+0.1N, eps 1e-6, W [768,3072] N(0,1/768)."""
    x = synth.normal_bf16((128, 768), 21)
    g = synth.normal_bf16((768,), 22, 0.1, 1.0)
    w = synth.normal_bf16((768, 3072), 23, 1.0 / np.sqrt(768))
    got = from_dev(K().fused_rmsnorm_matmul(to_dev(x), to_dev(w), to_dev(g), 1e-6))
    want = oracle.fused_rmsnorm_matmul(x, w, g, 1e-6)
    rep = mt.report(got, want)
    _say(f"config1: {rep}")
    assert rep.cosine >= 0.999 and rep.pcc >= 0.99 and rep.bit_exact >= 0.99, rep
    a = oracle.rmsnorm(x, g, 1e-6)
    assert _err_bound_ok(got, want, _abs_dot(a, w), 768, operand_ulps=1.0) == 0, rep


@pytest.mark.parametrize("M,N,Kd", [(64, 128, 64), (130, 200, 1600), (40, 96, 2048), (130, 200, 832),
                                    (33, 72, 128), (40, 96, 1024), (128, 4096, 768), (300, 4096, 768)])
def test_fused_rmsnorm_matmul_no_gamma(gpu, oracle, M, N, Kd):
    """K <= 832 and one round of 32 x 64 tiles: the latency-oriented panel
    kernel (ragged M and N); otherwise RMSNorm into workspace, then the GEMM."""
    x = synth.normal_bf16((M, Kd), 24)
    w = synth.normal_bf16((Kd, N), 25, 1.0 / np.sqrt(Kd))
    got = from_dev(K().fused_rmsnorm_matmul(to_dev(x), to_dev(w), None, 1e-5))
    want = oracle.fused_rmsnorm_matmul(x, w, None, 1e-5)
    rep = mt.report(got, want)
    assert rep.cosine >= 0.999 and rep.pcc >= 0.99 and rep.bit_exact >= 0.98, rep
    a = oracle.rmsnorm(x, None, 1e-5)
    assert _err_bound_ok(got, want, _abs_dot(a, w), Kd, operand_ulps=1.0) == 0, rep


@pytest.mark.parametrize("M,N,Kd", [(256, 512, 256), (130, 65, 127), (512, 2048, 1024)])
def test_fused_matmul_bias_gelu(gpu, oracle, M, N, Kd):
    a = synth.normal_bf16((M, Kd), 26)
    b = synth.normal_bf16((Kd, N), 27, 1.0 / np.sqrt(Kd))
    bias = synth.normal_bf16((N,), 28, 0.02)
    da, db, dbias = to_dev(a), to_dev(b), to_dev(bias)
    dgot = K().fused_matmul_bias_gelu(da, db, dbias)
    got = from_dev(dgot)
    want = oracle.fused_matmul_bias_gelu(a, b, bias)
    rep = mt.report(got, want)
    assert rep.cosine >= 0.999 and rep.pcc >= 0.99, rep
    assert rep.bit_exact >= 0.95, rep
    # every output is GELU(bf16(bf16(t) + bias)) for an fp32 accumulation t of the products
    assert _gate_bad(1, da, db, dgot, bias=dbias) == 0, rep
    assert _gate_bad(1, da, db, to_dev(want), bias=dbias) == 0  # the oracle's own order passes too


@pytest.mark.parametrize("tile", [0, 3])
def test_fused_matmul_bias_gelu_integer_bit_exact(gpu, oracle, tile):
    a, b = int_bf16((600, 384), 29), int_bf16((384, 520), 30)
    bias = bf(np.random.default_rng(31).integers(-4, 5, size=520))
    got = from_dev(K().gemm_ex(1, to_dev(a), to_dev(b), bias=to_dev(bias), tile=tile))
    assert np.array_equal(got, oracle.fused_matmul_bias_gelu(a, b, bias))


@pytest.mark.parametrize("tile", [0, 3])
def test_fused_matmul_bias_gelu_special_values_bit_exact(gpu, oracle, tile):
    # Rows of A that are all zero make bf16(bf16(acc) + bias) the bias itself, so the bias
    # row puts every special code through the epilogue: infinities, NaN, zeros of both
    # signs, the exponent-0/1 magnitudes the paired GELU hands to the per-element rules,
    # the largest finite values and the table edges.  The blocks that hold them take the
    # exact per-element path, the other blocks of the same launch the paired one.
    M, N, Kd = 512, 520, 96
    a, b = int_bf16((M, Kd), 36), int_bf16((Kd, N), 37)
    a[100:164] = 0
    a[480:] = 0
    bias = bf(np.random.default_rng(38).integers(-4, 5, size=N)).view(np.uint16).copy()
    special = [0x7F80, 0xFF80, 0x7FC0, 0xFFC0, 0x0000, 0x8000, 0x0001, 0x8001, 0x007F, 0x0080,
               0x80FF, 0x0100, 0x7F7F, 0xFF7F, 0x3B4A, 0x3B4B, 0xBB4B, 0x4031, 0x4032, 0xC0B1, 0xC0B2]
    cols = np.random.default_rng(39).choice(N, size=4 * len(special), replace=False)
    bias[cols] = np.tile(np.array(special, dtype=np.uint16), 4)
    bias = bias.view(a.dtype)
    got = from_dev(K().gemm_ex(1, to_dev(a), to_dev(b), bias=to_dev(bias), tile=tile))
    want = oracle.fused_matmul_bias_gelu(a, b, bias)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("tile", [0, 3])
def test_fused_matmul_bias_residual_integer_bit_exact(gpu, oracle, tile):
    a, b = int_bf16((600, 384), 32), int_bf16((384, 520), 33)
    bias = bf(np.random.default_rng(34).integers(-4, 5, size=520))
    r = rng_bf16((600, 520), 35)
    got = from_dev(K().gemm_ex(2, to_dev(a), to_dev(b), bias=to_dev(bias), residual=to_dev(r), tile=tile))
    assert np.array_equal(got, oracle.fused_matmul_bias_residual(a, b, bias, r))
    got = from_dev(K().fused_matmul_bias_residual(to_dev(a), to_dev(b), to_dev(bias), to_dev(r)))
    assert np.array_equal(got, oracle.fused_matmul_bias_residual(a, b, bias, r))
    got = from_dev(K().fused_matmul_bias_residual(to_dev(a), to_dev(b), None, to_dev(r)))
    assert np.array_equal(got, oracle.fused_matmul_bias_residual(a, b, None, r))


def _mlp_inputs(M, d, F):
    x = synth.normal_bf16((M, d), 40)
    g = synth.normal_bf16((d,), 41, 0.1, 1.0)
    w1 = synth.normal_bf16((d, F), 42, 1.0 / np.sqrt(d))
    b1 = synth.normal_bf16((F,), 43, 0.02)
    w2 = synth.normal_bf16((F, d), 44, 1.0 / np.sqrt(F))
    b2 = synth.normal_bf16((d,), 45, 0.02)
    return x, g, w1, b1, w2, b2


def test_mlp_block_small(gpu, oracle):
    x, g, w1, b1, w2, b2 = _mlp_inputs(256, 512, 2048)
    got = from_dev(K().mlp_block(*map(to_dev, (x, g, w1, b1, w2, b2)), eps=1e-6))
    want = oracle.mlp_block(x, g, w1, b1, w2, b2, 1e-6)
    rep = mt.report(got, want)
    assert rep.cosine >= 0.999 and rep.pcc >= 0.99 and rep.bit_exact >= 0.9, rep


def _bf16_ulp(v):
    """An upper bound on one bf16 ulp at magnitude |v| (and the subnormal step)."""
    return np.abs(v) * 2.0**-7 + 2.0**-133


def test_mlp_block_config2_row_sample(gpu, oracle):
    """Config 2 at full size on the GPU; rows are independent, so the oracle
    checks a seeded sample of 128 rows: the reference metrics on the block
    output, and a per-element error model of the block output against the
    oracle's whole chain.  With a = RMSNorm(x), t1 = bf16(bf16(a W1) + b1),
    h = GELU(t1), t2 = bf16(bf16(h W2) + b2), y = bf16(t2 + x), and bf16
    rounding monotone (|bf16(u) - bf16(v)| <= |u - v| + ulp):
      |dh| <= 1.13 (sum_k |da_k| |W1_k| + 2 K1 2^-23 sum |a| |W1| + 2 ulp(acc1) + ulp(t1)) + ulp(h)
      |dy| <= sum_k |dh_k| |W2_k| + 2 K2 2^-23 sum |h| |W2| + ulp(acc2) + ulp(t2) + ulp(y)
    (1.13 bounds |GELU'| on the real line; da and dh are the measured
    differences between the GPU's stages and the oracle's).  Any fp32
    summation order meets it; a wrong index, sign or dropped term does not."""
    import torch

    M, d, F = 4096, 4096, 16384
    _say("mlp_block config2 full")
    x, g, w1, b1, w2, b2 = _mlp_inputs(M, d, F)
    dx, dg, dw1, db1, dw2, db2 = map(to_dev, (x, g, w1, b1, w2, b2))
    block = K().mlp_block(dx, dg, dw1, db1, dw2, db2, eps=1e-6)
    rows = np.sort(np.random.default_rng(46).choice(M, 128, replace=False))
    trows = torch.from_numpy(rows).cuda()
    pick = lambda t: from_dev(t.index_select(0, trows).contiguous())
    got = pick(block)
    # the GPU's stages (the block is their chain, bit for bit)
    da_ = K().rmsnorm(dx, dg, 1e-6)
    dh_ = K().fused_matmul_bias_gelu(da_, dw1, db1)
    dy_ = K().fused_matmul_bias_residual(dh_, dw2, db2, dx)
    torch.cuda.synchronize()
    assert torch.equal(block.view(torch.int16), dy_.view(torch.int16))
    ga, gh = pick(da_), pick(dh_)
    del da_, dh_, dy_, block
    # the oracle's chain on the sample, which is its mlp_block
    xs = x[rows]
    oa = oracle.rmsnorm(xs, g, 1e-6)
    oh = oracle.fused_matmul_bias_gelu(oa, w1, b1)
    want = oracle.fused_matmul_bias_residual(oh, w2, b2, xs)
    assert np.array_equal(want, oracle.mlp_block(xs, g, w1, b1, w2, b2, 1e-6))
    rep = mt.report(got, want)
    _say(f"mlp config2 sample (128 rows): {rep}")
    assert rep.cosine >= 0.999 and rep.pcc >= 0.99 and rep.bit_exact >= 0.9, rep
    f = lambda b: f32(b).astype(np.float64)
    w1f, w2f = f(w1), f(w2)
    W1a, W2a = np.abs(w1f), np.abs(w2f)
    acc1 = f(oa) @ w1f
    dacc1 = np.abs(f(ga) - f(oa)) @ W1a + 2 * d * 2.0**-23 * (np.maximum(np.abs(f(ga)), np.abs(f(oa))) @ W1a)
    t1 = f(oracle.bias(oracle.matmul(oa, w1), b1))
    hmax = np.maximum(np.abs(f(gh)), np.abs(f(oh)))
    # + 2^-18 |h|: the reference GELU's own fp32 rounding before its bf16 rounding
    bh = 1.13 * (dacc1 + 2 * _bf16_ulp(np.abs(acc1) + dacc1) + _bf16_ulp(np.abs(t1) + dacc1 + _bf16_ulp(acc1))) \
        + _bf16_ulp(hmax) + 2.0**-18 * hmax
    dh = np.abs(f(gh) - f(oh))
    assert int((dh > bh).sum()) == 0, "h outside its error model"
    del acc1, dacc1, t1, bh, w1f, W1a
    acc2 = f(oh) @ w2f
    dacc2 = dh @ W2a + 2 * F * 2.0**-23 * (hmax @ W2a)
    t2 = acc2 + f(b2)
    by = dacc2 + 2 * _bf16_ulp(np.abs(acc2) + dacc2) + _bf16_ulp(np.abs(t2) + 2 * dacc2) \
        + _bf16_ulp(np.abs(t2 + f(xs)) + 3 * dacc2)
    bad = int((np.abs(f(got) - f(want)) > by).sum())
    assert bad == 0, (bad, rep)


def test_mlp_block_config2_stages_error_model(gpu, oracle):
    """Config 2 stage by stage at full size: RMSNorm, GEMM1 + bias + GELU,
    GEMM2 + bias + residual, each GEMM checked on a row sample against the fp32
    error model given the GPU's own previous stage (pk_gate_matmul: every
    output is the reference epilogue of some fp32 accumulation of its
    products); the stages chained give launch_mlp_block's bits."""
    import torch

    M, d, F = 4096, 4096, 16384
    _say("mlp config2 stages")
    x, g, w1, b1, w2, b2 = _mlp_inputs(M, d, F)
    dx, dg, dw1, db1, dw2, db2 = map(to_dev, (x, g, w1, b1, w2, b2))
    a = K().rmsnorm(dx, dg, 1e-6)
    h = K().fused_matmul_bias_gelu(a, dw1, db1)
    y = K().fused_matmul_bias_residual(h, dw2, db2, dx)
    block = K().mlp_block(dx, dg, dw1, db1, dw2, db2, eps=1e-6)
    torch.cuda.synchronize()
    assert torch.equal(block.view(torch.int16), y.view(torch.int16))
    rows = torch.from_numpy(np.sort(np.random.default_rng(47).choice(M, 16, replace=False))).cuda()
    pick = lambda t: t.index_select(0, rows).contiguous()
    ra = from_dev(pick(a))
    rep = mt.report(ra, oracle.rmsnorm(x[rows.cpu().numpy()], g, 1e-6))
    assert rep.bit_exact >= 0.99 and rep.max_ulp <= 1, rep
    assert _gate_bad(1, pick(a), dw1, pick(h), bias=db1) == 0
    assert _gate_bad(2, pick(h), dw2, pick(y), bias=db2, r=pick(dx)) == 0


# ------------------------------------------------------------------ int8

@pytest.mark.parametrize("M,N,Kd", [(128, 128, 128), (256, 128, 256), (192, 160, 224), (130, 127, 65),
                                    (16, 28672, 8192), (16, 8192, 28672), (1, 64, 32)])
def test_matmul_int8(gpu, oracle, M, N, Kd):
    _say(f"int8 {M}x{N}x{Kd}")
    a = synth.normal_bf16((M, Kd), 50)
    wq, s = oracle.quantize_per_channel(synth.normal_bf16((Kd, N), 51, 1.0 / np.sqrt(Kd)))
    got = from_dev(K().matmul_int8(to_dev(a), to_dev(wq), to_dev(s)))
    want = oracle.matmul_int8(a, wq, s)
    rep = mt.report(got, want)
    _say(f"int8 {M}x{N}x{Kd}: {rep}")
    assert rep.cosine >= 0.999 and rep.pcc >= 0.99 and rep.bit_exact >= 0.99, rep
    wdeq = bf(wq.astype(np.float32) * s[None, :])  # |w| to within 1 bf16 ulp, for the bound only
    assert _err_bound_ok(got, want, _abs_dot(a, wdeq) * (1 + 2.0**-7), Kd) == 0, rep


def test_matmul_int8_integer_bit_exact(gpu, oracle):
    a = int_bf16((16, 4096), 52)
    wq = np.random.default_rng(53).integers(-127, 128, size=(4096, 1024)).astype(np.int8)
    s = np.full(1024, 0.25, np.float32)  # power of two: exact scaling
    got = from_dev(K().matmul_int8(to_dev(a), to_dev(wq), to_dev(s)))
    assert np.array_equal(got, oracle.matmul_int8(a, wq, s))


# Variants of the streaming int8 kernel (block_m, block_n, num_warps, stages):
# every instantiation the library carries (block_n = 16 * NT * waves).
_I8S_VARIANTS = [(16, 512, 4, 3), (16, 448, 4, 3), (16, 256, 2, 6), (16, 256, 4, 6), (16, 512, 8, 3),
                 (16, 512, 2, 4), (16, 128, 4, 6), (16, 64, 4, 6), (16, 448, 4, 4),
                 (32, 512, 4, 3), (32, 256, 4, 4), (32, 128, 4, 6),
                 (64, 512, 4, 2), (64, 256, 4, 3), (64, 128, 4, 3)]


@pytest.mark.parametrize("bm,bn,waves,stages", _I8S_VARIANTS)
@pytest.mark.parametrize("block_k", [0, 192, 1024])
def test_matmul_int8_stream_variants_bit_exact(gpu, oracle, bm, bn, waves, stages, block_k):
    """Each variant, with the built-in K split and explicit ones (192 rows: 3
    steps, fewer than the ring depth; 1024 rows); N leaves a ragged last slice
    (and whole waves past N), M a ragged last m-tile."""
    M, N, Kd = bm - 3, 2 * bn + bn // 4 + 16, 1600 - 1600 % 64
    cfg = dict(block_m=bm, block_n=bn, block_k=block_k, num_warps=waves, shared_memory_stages=stages)
    _say(f"int8 stream {cfg} M={M} N={N} K={Kd}")
    a, wq, s = _int8_exact_inputs(M, N, Kd, 70)
    got = from_dev(K().matmul_int8_ex(0, to_dev(a), to_dev(wq), to_dev(s), config=cfg))
    assert np.array_equal(got, oracle.matmul_int8(a, wq, s))


@pytest.mark.parametrize("M,N,Kd", [(1, 16, 64), (5, 112, 64), (16, 1024, 128), (17, 2048, 4096),
                                    (64, 4096, 1024), (65, 256, 512), (130, 512, 256),
                                    (16, 28672, 512), (16, 8192, 1024)])
def test_matmul_int8_default_config_bit_exact(gpu, oracle, M, N, Kd):
    cfg = K().int8_default_config(M, N, Kd)
    _say(f"int8 default {M}x{N}x{Kd}: {cfg}")
    assert cfg is not None
    a, wq, s = _int8_exact_inputs(M, N, Kd, 71)
    got = from_dev(K().matmul_int8(to_dev(a), to_dev(wq), to_dev(s)))
    assert np.array_equal(got, oracle.matmul_int8(a, wq, s))


@pytest.mark.parametrize("cfg", [None, dict(block_m=16, block_n=256, block_k=256, num_warps=4,
                                            shared_memory_stages=6)])
def test_matmul_int8_epilogues_bit_exact(gpu, oracle, cfg):
    """GELU and residual epilogues, direct and through the split reduction."""
    M, N, Kd = 16, 1024, 1024
    a, wq, s = _int8_exact_inputs(M, N, Kd, 72)
    r = rng_bf16((M, N), 73)
    plain = oracle.matmul_int8(a, wq, s)
    got_g = from_dev(K().matmul_int8_ex(1, to_dev(a), to_dev(wq), to_dev(s), config=cfg))
    assert np.array_equal(got_g, oracle.gelu(plain))
    got_r = from_dev(K().matmul_int8_ex(2, to_dev(a), to_dev(wq), to_dev(s), residual=to_dev(r),
                                        config=cfg))
    assert np.array_equal(got_r, oracle.add(plain, r))


def test_matmul_int8_unsupported_config(gpu):
    from polykernel_amd._lib import PK_ERR_UNSUPPORTED, PolyKernelError

    a = to_dev(int_bf16((16, 256), 74))
    wq = to_dev(np.zeros((256, 192), np.int8))
    s = to_dev(np.ones(192, np.float32))
    for cfg in (dict(block_n=96), dict(block_n=1024), dict(block_k=100), dict(block_m=48), dict(num_warps=3)):
        with pytest.raises(PolyKernelError) as e:
            K().matmul_int8_ex(0, a, wq, s, config=cfg)
        assert e.value.code == PK_ERR_UNSUPPORTED


def test_decode_mlp_int8_config5(gpu, oracle):
    M, d, F = 16, 8192, 28672
    _say("decode int8 config5")
    x = synth.normal_bf16((M, d), 60)
    w1 = synth.normal_bf16((d, F), 61, 1.0 / np.sqrt(d))
    w2 = synth.normal_bf16((F, d), 62, 1.0 / np.sqrt(F))
    w1q, s1 = K().quantize_per_channel(to_dev(w1))
    w2q, s2 = K().quantize_per_channel(to_dev(w2))
    got = from_dev(K().decode_mlp_int8(to_dev(x), w1q, s1, w2q, s2))
    ow1q, os1 = oracle.quantize_per_channel(w1)
    ow2q, os2 = oracle.quantize_per_channel(w2)
    assert np.array_equal(from_dev(w1q), ow1q) and np.array_equal(from_dev(s2), os2)
    want = oracle.decode_mlp_int8(x, ow1q, os1, ow2q, os2)
    rep = mt.report(got, want)
    _say(f"decode config5: {rep}")
    assert rep.cosine >= 0.999 and rep.pcc >= 0.99 and rep.bit_exact >= 0.9, rep
    # stage by stage against the fp32 error model given the GPU's own h
    dx = to_dev(x)
    h = K().matmul_int8_ex(1, dx, w1q, s1)
    y = K().matmul_int8_ex(2, h, w2q, s2, residual=dx)
    assert np.array_equal(from_dev(y), got)  # the chain is launch_decode_mlp_int8's
    assert _gate_int8_bad(1, dx, w1q, s1, h) == 0
    assert _gate_int8_bad(2, h, w2q, s2, y, r=dx) == 0


# ------------------------------------------------------------------ attention

@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("B,H,Sq,Skv,D", [(1, 2, 32, 32, 32), (2, 4, 16, 16, 64), (1, 1, 24, 24, 40),
                                          (1, 2, 33, 33, 32), (1, 2, 128, 128, 64), (1, 2, 100, 300, 128)])
def test_attention_prefill(gpu, oracle, B, H, Sq, Skv, D, causal):
    _say(f"attention {B},{H},{Sq},{Skv},{D} causal={causal}")
    q, k, v = rng_bf16((B, H, Sq, D), 70), rng_bf16((B, H, Skv, D), 71), rng_bf16((B, H, Skv, D), 72)
    got = from_dev(K().attention_prefill(to_dev(q), to_dev(k), to_dev(v), None, causal))
    want = oracle.attention_prefill(q, k, v, None, causal)
    rep = mt.report(got, want)
    _say(f"attention: {rep}")
    assert rep.cosine >= 0.999 and rep.pcc >= 0.99 and rep.bit_exact >= 0.9, rep
    assert _att_bound_bad(oracle, got, want, q, k, v, causal) == 0, rep


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("B,H,Sq,Skv,D", [(1, 64, 128, 128, 64), (2, 32, 130, 400, 128),
                                          (1, 128, 64, 64, 128), (1, 128, 200, 1000, 64),
                                          (1, 4, 64, 4096, 64), (1, 2, 200, 2100, 128)])
def test_attention_prefill_flash_path(gpu, oracle, B, H, Sq, Skv, D, causal):
    """Head dims 64 and 128 take the flash-style kernel: ragged query and key
    counts (not multiples of 128 / 64), and small grids whose key range is
    split over up to 8 workgroups and merged by the combine kernel."""
    _say(f"attention flash {B},{H},{Sq},{Skv},{D} causal={causal}")
    q, k, v = rng_bf16((B, H, Sq, D), 90), rng_bf16((B, H, Skv, D), 91), rng_bf16((B, H, Skv, D), 92)
    got = from_dev(K().attention_prefill(to_dev(q), to_dev(k), to_dev(v), None, causal))
    want = oracle.attention_prefill(q, k, v, None, causal)
    rep = mt.report(got, want)
    _say(f"attention flash: {rep}")
    assert rep.cosine >= 0.999 and rep.pcc >= 0.99 and rep.bit_exact >= 0.9, rep
    assert _att_bound_bad(oracle, got, want, q, k, v, causal) == 0, rep


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("B,H,Sq,Skv,D", [(1, 2, 100, 300, 256), (2, 2, 64, 200, 200), (1, 1, 33, 70, 190),
                                          (1, 1, 32, 2048, 256), (1, 3, 130, 130, 160)])
def test_attention_prefill_wide_heads(gpu, oracle, B, H, Sq, Skv, D, causal):
    """Head dims above 128 up to 256 (the generic kernel at DP = 256): aligned
    and unaligned D, ragged tiles, and a one-tile grid whose key range is
    split and merged."""
    _say(f"attention wide {B},{H},{Sq},{Skv},{D} causal={causal}")
    q, k, v = rng_bf16((B, H, Sq, D), 76), rng_bf16((B, H, Skv, D), 77), rng_bf16((B, H, Skv, D), 78)
    got = from_dev(K().attention_prefill(to_dev(q), to_dev(k), to_dev(v), None, causal))
    want = oracle.attention_prefill(q, k, v, None, causal)
    rep = mt.report(got, want)
    _say(f"attention wide: {rep}")
    assert rep.cosine >= 0.999 and rep.pcc >= 0.99 and rep.bit_exact >= 0.9, rep
    assert _att_bound_bad(oracle, got, want, q, k, v, causal) == 0, rep


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("B,H,Sq,Skv,D", [(1, 2, 100, 300, 512), (2, 2, 64, 200, 320), (1, 1, 33, 70, 300),
                                          (1, 1, 32, 1024, 1024), (1, 3, 65, 130, 1000), (1, 1, 40, 40, 264)])
def test_attention_prefill_head_dims_above_256(gpu, oracle, B, H, Sq, Skv, D, causal):
    """Head dims 257..1024 (attention_prefill.cu:166-180 accepts D <= 1024):
    the wide kernel splits the dims over its 4 waves (one to four of them
    active), aligned and unaligned D (300), ragged query and key counts, and a
    one-tile grid whose key range is split over 8 workgroups and merged."""
    _say(f"attention D>256 {B},{H},{Sq},{Skv},{D} causal={causal}")
    q, k, v = rng_bf16((B, H, Sq, D), 86), rng_bf16((B, H, Skv, D), 87), rng_bf16((B, H, Skv, D), 88)
    got = from_dev(K().attention_prefill(to_dev(q), to_dev(k), to_dev(v), None, causal))
    want = oracle.attention_prefill(q, k, v, None, causal)
    rep = mt.report(got, want)
    _say(f"attention D>256: {rep}")
    assert rep.cosine >= 0.999 and rep.pcc >= 0.99 and rep.bit_exact >= 0.9, rep
    assert _att_bound_bad(oracle, got, want, q, k, v, causal) == 0, rep


def test_attention_head_dim_above_1024_refused(gpu):
    from polykernel_amd._lib import PK_ERR_UNSUPPORTED, PolyKernelError

    q = to_dev(rng_bf16((1, 1, 8, 1032), 79))
    with pytest.raises(PolyKernelError) as e:
        K().attention_prefill(q, q, q, None, True)
    assert e.value.code == PK_ERR_UNSUPPORTED and "1024" in e.value.message


@pytest.mark.parametrize("Sc,D", [(192, 128), (201, 128), (128, 64), (130, 64), (160, 256), (96, 384)])
def test_fused_kv_append_attention_flash_path(gpu, oracle, Sc, D):
    """In-place append fused into the flash kernel (S_cache a multiple of its
    64-key step) and the fallback (separate append kernels) otherwise; the
    cache is checked bit-exactly, including the rows past S_cache + S_q that
    must stay untouched."""
    import torch

    B, H, Sq = 2, 32, 70
    _say(f"fused append flash Sc={Sc} D={D}")
    q = rng_bf16((B, H, Sq, D), 93)
    kn, vn = rng_bf16((B, H, Sq, D), 94), rng_bf16((B, H, Sq, D), 95)
    kc, vc = rng_bf16((B, H, Sc, D), 96), rng_bf16((B, H, Sc, D), 97)
    cap = Sc + Sq + 5
    kcd = torch.full((B, H, cap, D), 7.0, dtype=torch.bfloat16, device="cuda")
    vcd = torch.full_like(kcd, -3.0)
    kcd[:, :, :Sc] = to_dev(kc)
    vcd[:, :, :Sc] = to_dev(vc)
    got = from_dev(K().fused_kv_append_attention(to_dev(q), to_dev(kn), to_dev(vn), kcd, vcd, Sc))
    kfull, vfull = oracle.kv_append(kc, kn), oracle.kv_append(vc, vn)
    kd, vd = from_dev(kcd), from_dev(vcd)
    assert np.array_equal(kd[:, :, :Sc + Sq], kfull) and np.array_equal(vd[:, :, :Sc + Sq], vfull)
    assert np.all(kd[:, :, Sc + Sq:] == bf([7.0])[0]) and np.all(vd[:, :, Sc + Sq:] == bf([-3.0])[0])
    want = oracle.attention_prefill(q, kfull, vfull, None, True)
    rep = mt.report(got, want)
    _say(f"fused append flash: {rep}")
    assert rep.cosine >= 0.999 and rep.pcc >= 0.99 and rep.bit_exact >= 0.9, rep
    assert _att_bound_bad(oracle, got, want, q, kfull, vfull, True) == 0, rep


@pytest.mark.parametrize("D", [128, 96, 512])
def test_attention_known_answers(gpu, D):
    """Closed forms on the device, no oracle: one key gives O = V bit for bit;
    zero keys give uniform weights, so O is the mean of the visible V (exact
    when the count is a power of two, within one bf16 ulp otherwise); causal
    outputs do not move when future keys and values change.  D 128 takes the
    flash kernel, 96 the generic one, 512 the wide one."""
    from polykernel_amd.synth import f32_to_bf16

    def run(q, k, v, causal):
        return from_dev(K().attention_prefill(to_dev(q), to_dev(k), to_dev(v), None, causal))

    q, k, v = rng_bf16((1, 4, 1, D), 80), rng_bf16((1, 4, 1, D), 81), rng_bf16((1, 4, 1, D), 82)
    for causal in (False, True):
        assert np.array_equal(run(q, k, v, causal), v), (D, causal)
    # zero keys: non-causal over 64 keys (mean exact), causal over i + 1 keys
    q = rng_bf16((1, 2, 16, D), 83)
    k = np.zeros((1, 2, 64, D), np.uint16)
    v = int_bf16((1, 2, 64, D), 84)
    want = f32_to_bf16((f32(v).astype(np.float64).sum(axis=2, keepdims=True) / 64).astype(np.float32))
    assert np.array_equal(run(q, k, v, False), np.broadcast_to(want, (1, 2, 16, D))), D
    n = 40
    q, k, v = rng_bf16((1, 2, n, D), 85), np.zeros((1, 2, n, D), np.uint16), int_bf16((1, 2, n, D), 86)
    got = f32(run(q, k, v, True)).astype(np.float64)
    csum = np.cumsum(f32(v).astype(np.float64), axis=2)
    cnt = np.arange(1, n + 1, dtype=np.float64)[None, None, :, None]
    mean = csum / cnt
    ulp = np.maximum(np.abs(mean), 2.0**-126) * 2.0**-7
    assert np.all(np.abs(got - mean) <= ulp), D
    pow2 = np.array([(i + 1) & i == 0 for i in range(n)])
    assert np.array_equal(got[:, :, pow2], f32(f32_to_bf16(mean[:, :, pow2].astype(np.float32)))), D
    # future keys and values do not reach earlier queries
    n, cut = 100, 60
    q, k, v = rng_bf16((1, 2, n, D), 87), rng_bf16((1, 2, n, D), 88), rng_bf16((1, 2, n, D), 89)
    k2, v2 = k.copy(), v.copy()
    k2[:, :, cut:], v2[:, :, cut:] = rng_bf16((1, 2, n - cut, D), 90), rng_bf16((1, 2, n - cut, D), 91)
    a, b = run(q, k, v, True), run(q, k2, v2, True)
    assert np.array_equal(a[:, :, :cut], b[:, :, :cut]), D
    assert not np.array_equal(a[:, :, cut:], b[:, :, cut:]), D


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("H,Skv,D", [(8, 777, 128), (8, 4096, 64), (4, 2000, 96), (2, 1500, 512)])
def test_attention_single_query(gpu, oracle, H, Skv, D, causal):
    """One query over a long key range (a decode step): the grid is one query
    tile per head, so the key range is split over workgroups and merged."""
    _say(f"attention single query H={H} Skv={Skv} D={D} causal={causal}")
    q, k, v = rng_bf16((1, H, 1, D), 92), rng_bf16((1, H, Skv, D), 93), rng_bf16((1, H, Skv, D), 94)
    got = from_dev(K().attention_prefill(to_dev(q), to_dev(k), to_dev(v), None, causal))
    want = oracle.attention_prefill(q, k, v, None, causal)
    rep = mt.report(got, want)
    assert rep.cosine >= 0.999 and rep.pcc >= 0.99 and rep.bit_exact >= 0.9, rep
    assert _att_bound_bad(oracle, got, want, q, k, v, causal) == 0, rep


def test_attention_leaky_mask_is_detected(gpu, oracle):
    q, k, v = rng_bf16((1, 2, 64, 64), 73), rng_bf16((1, 2, 64, 64), 74), rng_bf16((1, 2, 64, 64), 75)
    leak = from_dev(K().attention_prefill(to_dev(q), to_dev(k), to_dev(v), None, False))
    want = oracle.attention_prefill(q, k, v, None, True)
    assert not mt.report(leak, want).passes()


def test_fused_kv_append_attention_config3_heads(gpu, oracle):
    """Config 3 geometry (H=32, D=128, 3584 cached + 512 new, in-place append);
    the oracle checks all 32 heads plus the appended cache bit-exactly."""
    import torch

    B, H, Sc, Sn, D = 1, 32, 3584, 512, 128
    _say("attention config3")
    q = synth.normal_bf16((B, H, Sn, D), 80)
    kn, vn = synth.normal_bf16((B, H, Sn, D), 81), synth.normal_bf16((B, H, Sn, D), 82)
    kc, vc = synth.normal_bf16((B, H, Sc, D), 83), synth.normal_bf16((B, H, Sc, D), 84)
    cap = Sc + Sn
    kcd = torch.zeros(B, H, cap, D, dtype=torch.bfloat16, device="cuda")
    vcd = torch.zeros_like(kcd)
    kcd[:, :, :Sc] = to_dev(kc)
    vcd[:, :, :Sc] = to_dev(vc)
    got = from_dev(K().fused_kv_append_attention(to_dev(q), to_dev(kn), to_dev(vn), kcd, vcd, Sc))
    kfull, vfull = oracle.kv_append(kc, kn), oracle.kv_append(vc, vn)
    assert np.array_equal(from_dev(kcd), kfull) and np.array_equal(from_dev(vcd), vfull)
    heads = list(range(H))
    want = oracle.attention_prefill(q[:, heads], kfull[:, heads], vfull[:, heads], None, True)
    rep = mt.report(got[:, heads], want)
    _say(f"attention config3 heads {heads}: {rep}")
    assert rep.cosine >= 0.999 and rep.pcc >= 0.99 and rep.bit_exact >= 0.9, rep
    assert _att_bound_bad(oracle, got[:, heads], want, q[:, heads], kfull[:, heads], vfull[:, heads],
                          True) == 0, rep


@pytest.mark.parametrize("Sc,Sn,D", [(256, 160, 128), (384, 100, 64), (100, 60, 512)])
def test_fused_kv_append_attention_every_config(gpu, oracle, Sc, Sn, D):
    """Each configuration pk_op_configs lists (the flash kernel's 128 x 64 and
    64 x 128 tile shapes for D 64 / 128; the wide kernel's 32 x 32 for D 512)
    through pk_fused_kv_append_attention_config: the appended cache
    bit-exact, outputs within the attention error model."""
    import ctypes

    import torch

    from polykernel_amd import _lib

    lib = _lib.load()
    B, H = 1, 4
    cfgs = (_lib.Config * 8)()
    n = lib.pk_op_configs(b"fused_kv_append_attention", Sn, Sc + Sn, D, cfgs, 8)
    shapes = {(128, 64), (64, 128)} if D in (64, 128) else {(32, 32)}
    assert n == len(shapes), n
    assert {(cfgs[i].block_m, cfgs[i].block_n) for i in range(n)} == shapes
    q = rng_bf16((B, H, Sn, D), 110)
    kn, vn = rng_bf16((B, H, Sn, D), 111), rng_bf16((B, H, Sn, D), 112)
    kc, vc = rng_bf16((B, H, Sc, D), 113), rng_bf16((B, H, Sc, D), 114)
    kfull, vfull = oracle.kv_append(kc, kn), oracle.kv_append(vc, vn)
    want = oracle.attention_prefill(q, kfull, vfull, None, True)
    dq, dkn, dvn = to_dev(q), to_dev(kn), to_dev(vn)
    st = torch.cuda.current_stream().cuda_stream
    for i in range(n):
        c = cfgs[i]
        _say(f"fused append config {c.block_m}x{c.block_n} Sc={Sc} Sn={Sn} D={D}")
        kcd = torch.zeros(B, H, Sc + Sn, D, dtype=torch.bfloat16, device="cuda")
        vcd = torch.zeros_like(kcd)
        kcd[:, :, :Sc] = to_dev(kc)
        vcd[:, :, :Sc] = to_dev(vc)
        out = torch.empty(B, H, Sn, D, dtype=torch.bfloat16, device="cuda")
        _lib.check(lib.pk_fused_kv_append_attention_config(
            dq.data_ptr(), kcd.data_ptr(), vcd.data_ptr(), dkn.data_ptr(), dvn.data_ptr(), out.data_ptr(),
            B, H, Sn, Sc, D, Sc + Sn, 1.0 / np.sqrt(D), 1, ctypes.byref(c), st), "attention config")
        got = from_dev(out)
        assert np.array_equal(from_dev(kcd), kfull) and np.array_equal(from_dev(vcd), vfull)
        rep = mt.report(got, want)
        _say(f"  {rep}")
        assert rep.cosine >= 0.999 and rep.pcc >= 0.99 and rep.bit_exact >= 0.9, rep
        assert _att_bound_bad(oracle, got, want, q, kfull, vfull, True) == 0, rep


def test_fused_kv_append_attention_config_errors(gpu):
    """A config outside the list is refused; the 64 x 128 tile shape refuses
    an S_cache that is not a multiple of its 128-key step (no launch)."""
    import ctypes

    import torch

    from polykernel_amd import _lib

    lib = _lib.load()
    B, H, Sn, Sc, D = 1, 2, 64, 192, 128
    t = lambda *s: torch.zeros(*s, dtype=torch.bfloat16, device="cuda")
    q, kn, vn, out = t(B, H, Sn, D), t(B, H, Sn, D), t(B, H, Sn, D), t(B, H, Sn, D)
    kc, vc = t(B, H, Sc + Sn, D), t(B, H, Sc + Sn, D)
    st = torch.cuda.current_stream().cuda_stream

    def run(c):
        return lib.pk_fused_kv_append_attention_config(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), kn.data_ptr(),
                                                       vn.data_ptr(), out.data_ptr(), B, H, Sn, Sc, D, Sc + Sn,
                                                       0.088, 1, ctypes.byref(c), st)

    assert run(_lib.Config(96, 64, 128, 8, 8, 8, 4)) == _lib.PK_ERR_INVALID_ARG
    assert "not a config" in _lib.last_error()
    cfgs = (_lib.Config * 8)()
    n = lib.pk_op_configs(b"fused_kv_append_attention", Sn, Sc + Sn, D, cfgs, 8)
    wide = [cfgs[i] for i in range(n) if cfgs[i].block_n == 128][0]
    assert run(wide) == _lib.PK_ERR_UNSUPPORTED
    assert "multiple of 128" in _lib.last_error()
    narrow = [cfgs[i] for i in range(n) if cfgs[i].block_n == 64][0]
    assert run(narrow) == 0
    torch.cuda.synchronize()


# ------------------------------------------------------------------ error paths

def test_invalid_arguments_return_status(gpu):
    from polykernel_amd import _lib

    lib = _lib.load()
    rc = lib.launch_rmsnorm(None, None, None, 4, 8, 1e-5, None)
    assert rc == _lib.PK_ERR_INVALID_ARG
    assert "null" in _lib.last_error()
    rc = lib.launch_mlp_block(1, None, 1, 1, 1, 1, 1, 4, 8, 8, 1e-5, None, 0, None)
    assert rc == _lib.PK_ERR_WORKSPACE
