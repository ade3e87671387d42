"""launch_matmul_int8_noalloc: the allocation-free variant of launch_matmul_int8.

Called through the C-ABI on two shapes in a row (the second smaller, so the
static scratch still holds the first call's partials), each compared bit for
bit with launch_matmul_int8 on the same inputs; the unaligned-shape path
(generic kernel) too; and the calls leave the device's free memory
unchanged.  (A shape whose split-K partials exceed the static buffer is
refused before any device call: tests/test_host_args.py checks that on the
CPU.)
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from tests.helpers import from_dev, rng_bf16, to_dev

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20


def _say(msg):
    print(msg, flush=True)


def _mem_free():
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def _case(M, N, Kd, seed):
    rng = np.random.default_rng(seed)
    a = rng_bf16((M, Kd), seed)
    wq = rng.integers(-127, 128, size=(Kd, N)).astype(np.int8)
    s = rng.uniform(0.001, 0.01, size=N).astype(np.float32)
    return to_dev(a), to_dev(wq), to_dev(s)


def _split_bytes(M, N, Kd):
    from polykernel_amd import runtime as rt

    cfg = rt.default_config("matmul_int8", M, N, Kd)
    if cfg is None:  # generic kernel
        return None
    splits = -(-Kd // cfg["block_k"])
    return splits * M * N * 4 if splits > 1 else 0


def test_noalloc_matches_launch_matmul_int8(gpu):
    import torch

    from polykernel_amd import _lib

    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    shapes = [(16, 8192, 28672), (16, 4096, 8192)]  # config-5 W2 shape, then a smaller one
    for M, N, Kd in shapes:
        need = _split_bytes(M, N, Kd)
        assert need is not None and 0 < need <= SCRATCH_BYTES, (M, N, Kd, need)
    cases = [_case(*sh, seed=50 + i) for i, sh in enumerate(shapes)]
    outs = [torch.empty((M, N), dtype=torch.bfloat16, device="cuda") for M, N, _ in shapes]
    refs = [torch.empty((M, N), dtype=torch.bfloat16, device="cuda") for M, N, _ in shapes]
    # set-up: loads the library's code object on this device (the static
    # scratch comes with it) and looks up the scratch's device address
    _lib.check(lib.pk_init(), "pk_init")
    torch.cuda.synchronize()
    before = _mem_free()
    for (M, N, Kd), (a, w, s), o in zip(shapes, cases, outs):
        _say(f"launch_matmul_int8_noalloc M={M} N={N} K={Kd}")
        _lib.check(lib.launch_matmul_int8_noalloc(a.data_ptr(), w.data_ptr(), s.data_ptr(), o.data_ptr(),
                                                  M, N, Kd, st), "launch_matmul_int8_noalloc")
    torch.cuda.synchronize()
    assert _mem_free() == before, "the no-allocation entry point changed the device's free memory"
    for (M, N, Kd), (a, w, s), r in zip(shapes, cases, refs):
        _lib.check(lib.launch_matmul_int8(a.data_ptr(), w.data_ptr(), s.data_ptr(), r.data_ptr(), M, N, Kd, st),
                   "launch_matmul_int8")
    torch.cuda.synchronize()
    for o, r in zip(outs, refs):
        assert np.array_equal(from_dev(o), from_dev(r))


def test_noalloc_generic_kernel_path(gpu):
    """N not a multiple of 16: the generic int8 kernel, its split-K partials in
    the same static scratch."""
    import torch

    from polykernel_amd import _lib

    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    for M, N, Kd in [(16, 1000, 8192), (5, 72, 4104)]:
        a, w, s = _case(M, N, Kd, seed=M + N)
        o = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        r = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        _lib.check(lib.launch_matmul_int8_noalloc(a.data_ptr(), w.data_ptr(), s.data_ptr(), o.data_ptr(),
                                                  M, N, Kd, st), "noalloc")
        _lib.check(lib.launch_matmul_int8(a.data_ptr(), w.data_ptr(), s.data_ptr(), r.data_ptr(), M, N, Kd, st),
                   "launch_matmul_int8")
        torch.cuda.synchronize()
        assert np.array_equal(from_dev(o), from_dev(r)), (M, N, Kd)
