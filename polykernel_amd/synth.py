"""Deterministic synthetic inputs (host side).

Counter-based generator of the C-ABI (pk_synth_*): SplitMix64 -> Box-Muller in
double -> fp32 -> bf16 RNE.  Draw i of a (seed, stream) pair does not depend on
the thread count or on how the tensor is sliced, so a row sample of a large
tensor can be regenerated on its own.  N(mu, var) is read as a variance.
"""
from __future__ import annotations

import math

import numpy as np

from . import _lib

SEED = 0xC0FFEE


def normal_bf16(shape, stream: int, std: float = 1.0, mean: float = 0.0, seed: int = SEED) -> np.ndarray:
    """bf16 bits (np.uint16) of N(mean, std^2) draws."""
    out = np.empty(shape, dtype=np.uint16)
    _lib.load().pk_synth_normal_bf16(seed, stream, float(mean), float(std),
                                     out.ctypes.data, out.size)
    return out


def normal_f32(shape, stream: int, std: float = 1.0, mean: float = 0.0, seed: int = SEED) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    _lib.load().pk_synth_normal_f32(seed, stream, float(mean), float(std), out.ctypes.data, out.size)
    return out


def mask_bf16(shape, stream: int, p: float = 0.1, seed: int = SEED) -> np.ndarray:
    """Additive mask bits: -inf with probability p, else 0."""
    out = np.empty(shape, dtype=np.uint16)
    _lib.load().pk_synth_mask_bf16(seed, stream, float(p), out.ctypes.data, out.size)
    return out


def fan_in_std(fan_in: int) -> float:
    """sigma of N(0, 1/fan_in)."""
    return 1.0 / math.sqrt(fan_in)


# ---- bf16 <-> fp32 on the host (numpy), RNE with NaN -> quiet NaN ----------

def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = ((u & 0x7F800000) == 0x7F800000) & ((u & 0x007FFFFF) != 0)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    q = ((u >> 16) | 0x0040).astype(np.uint16)
    return np.where(nan, q, r)


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
