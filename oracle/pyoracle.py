"""ctypes binding of the C oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  numpy uint16 arrays carry bf16
bits.  Also binds the reference's own kernels/cpu build (oracle/_ref) when it
exists (this container only).
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liboracle.so"
REF_DIR = HERE / "_ref"

P, I64, F = C.c_void_p, C.c_int64, C.c_float

_SIGS = {
    "pko_f32_to_bf16": (C.c_uint16, [F]),
    "pko_f32_to_bf16_array": (None, [P, P, I64]),
    "pko_rmsnorm": (None, [P, P, P, I64, I64, F]),
    "pko_add": (None, [P, P, P, I64]),
    "pko_bias": (None, [P, P, P, I64, I64]),
    "pko_residual_rmsnorm": (None, [P, P, P, P, I64, I64, F]),
    "pko_gelu": (None, [P, P, I64]),
    "pko_matmul": (None, [P, P, P, I64, I64, I64]),
    "pko_fused_rmsnorm_matmul": (None, [P, P, P, P, I64, I64, I64, F]),
    "pko_fused_matmul_bias_gelu": (None, [P, P, P, P, I64, I64, I64]),
    "pko_fused_matmul_bias_residual": (None, [P, P, P, P, P, I64, I64, I64]),
    "pko_softmax": (None, [P, P, I64, I64]),
    "pko_softmax_mask": (None, [P, P, P, I64, I64]),
    "pko_kv_append": (None, [P, P, P, I64, I64, I64, I64]),
    "pko_attention_prefill": (None, [P, P, P, P, I64, I64, I64, I64, F, C.c_int]),
    "pko_quantize_per_channel": (None, [P, P, P, I64, I64]),
    "pko_matmul_int8": (None, [P, P, P, P, I64, I64, I64]),
    "pko_mlp_block": (None, [P, P, P, P, P, P, P, I64, I64, I64, F]),
    "pko_decode_mlp_int8": (None, [P, P, P, P, P, P, I64, I64, I64]),
    "pko_num_threads": (C.c_int, []),
    "pko_set_num_threads": (None, [C.c_int]),
}

_lib = None


def build() -> None:
    """Compile the C oracle (and the reference build when /root/reference exists)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    if Path("/root/reference/kernels/cpu/cpu_reference.cpp").exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "ref"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        l = C.CDLL(str(LIB))
        for n, (r, a) in _SIGS.items():
            fn = getattr(l, n)
            fn.restype, fn.argtypes = r, a
        _lib = l
    return _lib


def _p(a):
    return None if a is None else np.ascontiguousarray(a).ctypes.data


def _u16(a):
    return np.ascontiguousarray(a, dtype=np.uint16)


def num_threads() -> int:
    return lib().pko_num_threads()


def set_num_threads(n: int) -> None:
    lib().pko_set_num_threads(n)


def rmsnorm(x, w=None, eps=1e-5):
    x = _u16(x)
    out = np.empty_like(x)
    cols = x.shape[-1]
    lib().pko_rmsnorm(_p(x), _p(None if w is None else _u16(w)), _p(out), x.size // cols, cols, eps)
    return out


def add(a, b):
    a, b = _u16(a), _u16(b)
    out = np.empty_like(a)
    lib().pko_add(_p(a), _p(b), _p(out), a.size)
    return out


def bias(x, b):
    """golden.bias (tests/golden/golden.py:53-55): bf16(f32(x[i, j]) + f32(b[j]))."""
    x, b = _u16(x), _u16(b)
    out = np.empty_like(x)
    N = x.shape[-1]
    lib().pko_bias(_p(x), _p(b), _p(out), x.size // N, N)
    return out


def residual_rmsnorm(x, r, w=None, eps=1e-5):
    x, r = _u16(x), _u16(r)
    out = np.empty_like(x)
    cols = x.shape[-1]
    lib().pko_residual_rmsnorm(_p(x), _p(r), _p(None if w is None else _u16(w)), _p(out),
                               x.size // cols, cols, eps)
    return out


def gelu(x):
    x = _u16(x)
    out = np.empty_like(x)
    lib().pko_gelu(_p(x), _p(out), x.size)
    return out


def matmul(a, b):
    a, b = _u16(a), _u16(b)
    K = a.shape[-1]
    M, N = a.size // K, b.shape[1]
    out = np.empty(a.shape[:-1] + (N,), dtype=np.uint16)
    lib().pko_matmul(_p(a), _p(b), _p(out), M, N, K)
    return out


def fused_rmsnorm_matmul(x, w, gamma=None, eps=1e-5):
    x, w = _u16(x), _u16(w)
    K = x.shape[-1]
    M, N = x.size // K, w.shape[1]
    out = np.empty(x.shape[:-1] + (N,), dtype=np.uint16)
    g = None if gamma is None else _u16(gamma)
    lib().pko_fused_rmsnorm_matmul(_p(x), _p(g), _p(w), _p(out), M, N, K, eps)
    return out


def fused_matmul_bias_gelu(a, b, bias):
    a, b, bias = _u16(a), _u16(b), _u16(bias)
    K = a.shape[-1]
    M, N = a.size // K, b.shape[1]
    out = np.empty(a.shape[:-1] + (N,), dtype=np.uint16)
    lib().pko_fused_matmul_bias_gelu(_p(a), _p(b), _p(bias), _p(out), M, N, K)
    return out


def fused_matmul_bias_residual(a, b, bias, residual):
    a, b, residual = _u16(a), _u16(b), _u16(residual)
    K = a.shape[-1]
    M, N = a.size // K, b.shape[1]
    out = np.empty(a.shape[:-1] + (N,), dtype=np.uint16)
    bb = None if bias is None else _u16(bias)
    lib().pko_fused_matmul_bias_residual(_p(a), _p(b), _p(bb), _p(residual), _p(out), M, N, K)
    return out


def softmax(x):
    x = _u16(x)
    out = np.empty_like(x)
    cols = x.shape[-1]
    lib().pko_softmax(_p(x), _p(out), x.size // cols, cols)
    return out


def softmax_mask(logits, mask):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    mask = _u16(mask)
    out = np.empty(logits.shape, dtype=np.uint16)
    cols = logits.shape[-1]
    lib().pko_softmax_mask(_p(logits), _p(mask), _p(out), logits.size // cols, cols)
    return out


def kv_append(cache, new):
    cache, new = _u16(cache), _u16(new)
    B, H, Sc, D = cache.shape
    Sn = new.shape[2]
    out = np.empty((B, H, Sc + Sn, D), dtype=np.uint16)
    lib().pko_kv_append(_p(cache), _p(new), _p(out), B * H, Sc, Sn, D)
    return out


def attention_prefill(q, k, v, scale=None, causal=True):
    q, k, v = _u16(q), _u16(k), _u16(v)
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    out = np.empty_like(q)
    lib().pko_attention_prefill(_p(q), _p(k), _p(v), _p(out), B * H, Sq, Skv, D, scale, int(causal))
    return out


def quantize_per_channel(w):
    w = _u16(w)
    K, N = w.shape
    wq = np.empty((K, N), dtype=np.int8)
    scale = np.empty(N, dtype=np.float32)
    lib().pko_quantize_per_channel(_p(w), _p(wq), _p(scale), K, N)
    return wq, scale


def matmul_int8(a, wq, scale):
    a = _u16(a)
    wq = np.ascontiguousarray(wq, dtype=np.int8)
    scale = np.ascontiguousarray(scale, dtype=np.float32)
    K = a.shape[-1]
    M, N = a.size // K, wq.shape[1]
    out = np.empty(a.shape[:-1] + (N,), dtype=np.uint16)
    lib().pko_matmul_int8(_p(a), _p(wq), _p(scale), _p(out), M, N, K)
    return out


def mlp_block(x, gamma, w1, b1, w2, b2, eps=1e-6):
    x = _u16(x)
    d = x.shape[-1]
    M, F_ = x.size // d, w1.shape[1]
    out = np.empty_like(x)
    g = None if gamma is None else _u16(gamma)
    lib().pko_mlp_block(_p(x), _p(g), _p(_u16(w1)), _p(_u16(b1)), _p(_u16(w2)), _p(_u16(b2)),
                        _p(out), M, d, F_, eps)
    return out


def decode_mlp_int8(x, w1q, s1, w2q, s2):
    x = _u16(x)
    d = x.shape[-1]
    M, F_ = x.size // d, w1q.shape[1]
    out = np.empty_like(x)
    lib().pko_decode_mlp_int8(_p(x), _p(np.ascontiguousarray(w1q, np.int8)),
                              _p(np.ascontiguousarray(s1, np.float32)),
                              _p(np.ascontiguousarray(w2q, np.int8)),
                              _p(np.ascontiguousarray(s2, np.float32)), _p(out), M, d, F_)
    return out


# ---- the reference's own kernels/cpu build (oracle/_ref), when present ------

def ref_available() -> bool:
    return (REF_DIR / "libpkref.so").exists()


_ref = None


def ref_lib():
    global _ref
    if _ref is None:
        l = C.CDLL(str(REF_DIR / "libpkref.so"))
        l.ref_rmsnorm.argtypes = [P, P, P, I64, I64, F]
        l.ref_gelu.argtypes = [P, P, I64]
        l.ref_matmul.argtypes = [P, P, P, I64, I64, I64]
        l.ref_fused_rmsnorm_matmul.argtypes = [P, P, P, I64, I64, I64, F]
        l.ref_fused_matmul_bias_gelu.argtypes = [P, P, P, P, I64, I64, I64]
        l.ref_softmax.argtypes = [P, P, I64, I64]
        l.ref_f32_to_bf16.argtypes = [F]
        l.ref_f32_to_bf16.restype = C.c_uint16
        _ref = l
    return _ref


def save_npy_bf16(path, bits: np.ndarray) -> None:
    """Write bf16 bits with the '<V2' void descr the reference's npy_io reads."""
    np.save(path, np.ascontiguousarray(bits, dtype=np.uint16).view("V2"))


def load_npy_bf16(path) -> np.ndarray:
    return np.load(path).view(np.uint16)


def run_ref(binary: str, *args) -> None:
    subprocess.run([str(REF_DIR / binary), *map(str, args)], check=True, capture_output=True)
