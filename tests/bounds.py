"""Error models and exact-input generators shared by the GPU parity tests:
per-element fp32 bounds for GEMM-class outputs (any fp32 summation order
passes them; a wrong index, sign or dropped term does not), the device gates
of the library's autotuner used as checkers, and integer-valued inputs on
which every summation order is exact."""
from __future__ import annotations

import numpy as np

from tests.helpers import f32, int_bf16


def _err_bound_ok(gpu_bits, ref_bits, abs_dot, Kdim, operand_ulps=0.0):
    """Number of outputs outside |gpu - ref| <= 2 ulp_bf16(ref) + (K 2^-23 + u 2^-8) sum|a||b|.

    K 2^-23 sum|a||b| bounds any fp32 summation order (two such sums differ by
    at most twice the classic gamma_K bound); u 2^-8 sum|a||b| admits u bf16 ulps
    of difference in each A operand (the fused RMSNorm prologue reduces the
    row sum of squares in a different order, so a normalised activation can
    round to the neighbouring bf16)."""
    g, r = f32(gpu_bits).astype(np.float64), f32(ref_bits).astype(np.float64)
    ulp = np.abs(r) * 2.0**-7 + 2.0**-133
    bound = 2 * ulp + (Kdim * 2.0**-23 + operand_ulps * 2.0**-8) * abs_dot
    bad = np.abs(g - r) > bound
    return int(bad.sum())


def _abs_dot(a_bits, b_bits):
    return np.abs(f32(a_bits).astype(np.float64)) @ np.abs(f32(b_bits).astype(np.float64))


def _gate_bad(epi, a, b, got, bias=None, r=None, operand_ulps=0.0):
    """Outputs outside the device fp32 error model (pk_gate_matmul): got must be
    the reference epilogue (bf16 GEMM epi 0 none, 1 bias+GELU, 2 bias+residual)
    applied to some fp32 accumulation of a @ b's products.  Arguments are
    device tensors (a row sample of A, R and got is enough: rows are
    independent)."""
    import ctypes

    import torch

    from polykernel_amd import _lib

    n = ctypes.c_ulonglong(0)
    M, Kd = a.shape
    N = b.shape[1]
    ptr = lambda t: None if t is None else t.data_ptr()
    _lib.check(_lib.load().pk_gate_matmul(epi, ptr(a), ptr(b), ptr(bias), ptr(r), ptr(got), M, N, Kd,
                                          float(operand_ulps), ctypes.byref(n),
                                          torch.cuda.current_stream().cuda_stream), "pk_gate_matmul")
    return n.value


def _gate_int8_bad(epi, a, wq, s, got, r=None):
    """As _gate_bad for the int8 weight-only GEMM (epi 0 none, 1 GELU, 2 residual)."""
    import ctypes

    import torch

    from polykernel_amd import _lib

    n = ctypes.c_ulonglong(0)
    M, Kd = a.shape
    N = wq.shape[1]
    _lib.check(_lib.load().pk_gate_matmul_int8(epi, a.data_ptr(), wq.data_ptr(), s.data_ptr(),
                                               None if r is None else r.data_ptr(), got.data_ptr(), M, N, Kd,
                                               ctypes.byref(n), torch.cuda.current_stream().cuda_stream),
               "pk_gate_matmul_int8")
    return n.value


def _int8_exact_inputs(M, N, Kd, seed):
    """Integer-valued activations, int8 weights, power-of-two scales: every
    partial sum is an integer below 2^24, so any summation order is exact and
    the GPU must match the oracle bit for bit."""
    a = int_bf16((M, Kd), seed, -4, 4)
    r = np.random.default_rng(seed + 1)
    wq = r.integers(-127, 128, size=(Kd, N)).astype(np.int8)
    s = (2.0 ** r.integers(-9, -4, size=N)).astype(np.float32)
    return a, wq, s


def _att_bound_bad(oracle, got, want, q, k, v, causal):
    """Outputs outside an fp32 error model of softmax attention.

    A weight w_j = exp(s_j - m) carries a relative error eps_w <= D 2^-23 scale
    max_j sum_d |q_d k_jd| (score summation order) + 2^-20 (exp) + 2^-16 (the
    bf16 hi/lo split of p); the output o = sum w v / sum w then moves by at most
    2 eps_w (sum w |v| / sum w + |o|), plus S_kv 2^-23 sum w |v| / sum w for the
    PV summation order, plus 2 bf16 ulp of the final rounding."""
    D, Skv = q.shape[-1], k.shape[2]
    scale = 1.0 / np.sqrt(D)
    qa = np.abs(f32(q).astype(np.float64))
    ka = np.abs(f32(k).astype(np.float64))
    max_qk = float(np.max(qa @ np.swapaxes(ka, -1, -2)))
    eps_w = D * 2.0**-23 * scale * max_qk + 2.0**-20 + 2.0**-16
    abs_att = f32(oracle.attention_prefill(q, k, v & 0x7FFF, None, causal)).astype(np.float64) * 1.01
    r = f32(want).astype(np.float64)
    g = f32(got).astype(np.float64)
    bound = 2 * (np.abs(r) * 2.0**-7 + 2.0**-133) + (2 * eps_w + Skv * 2.0**-23) * (abs_att + np.abs(r))
    return int((np.abs(g - r) > bound).sum())
