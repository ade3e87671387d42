"""Shared test helpers: device transfer of bf16 bit arrays, seeded inputs."""
from __future__ import annotations

import numpy as np


def to_dev(a: np.ndarray, dtype=None):
    import torch

    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).cuda()
    return torch.from_numpy(a).cuda()


def from_dev(t) -> np.ndarray:
    import torch

    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def rng_bf16(shape, seed: int, low=-1.0, high=1.0) -> np.ndarray:
    """uniform bf16 bits (numpy PCG64), RNE from fp32."""
    from polykernel_amd.synth import f32_to_bf16

    r = np.random.default_rng(seed)
    return f32_to_bf16(r.uniform(low, high, size=shape).astype(np.float32))


def int_bf16(shape, seed: int, lo=-3, hi=3) -> np.ndarray:
    """small integer values (exact in bf16; exact sums in any order)."""
    from polykernel_amd.synth import f32_to_bf16

    r = np.random.default_rng(seed)
    return f32_to_bf16(r.integers(lo, hi + 1, size=shape).astype(np.float32))


def bf(x) -> np.ndarray:
    from polykernel_amd.synth import f32_to_bf16

    return f32_to_bf16(np.asarray(x, dtype=np.float32))


def f32(b) -> np.ndarray:
    from polykernel_amd.synth import bf16_to_f32

    return bf16_to_f32(b)
