"""Re-entrancy of the launchers and large-operand addressing (GPU).

* Entry points whose reference signature has no workspace argument keep their
  split partials in library scratch owned per (device, stream): launches of
  split-K int8 and split-KV attention issued concurrently from two host
  threads on two streams, and two threads sharing one stream, give the bits
  of serial runs.
* The DMA GEMM addresses A through a buffer descriptor whose 32-bit record
  count covers only the tile's own 256 rows, so A operands of 4 GiB and more
  are read in full (integer inputs: bit-exact against the oracle on rows
  around the 2^32-byte boundary).
"""
from __future__ import annotations

import threading

import numpy as np
import pytest

from tests.helpers import from_dev, int_bf16, rng_bf16, to_dev

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _int8_case(seed, M=16, N=4096, Kd=8192):
    rng = np.random.default_rng(seed)
    a = rng_bf16((M, Kd), seed)
    wq = rng.integers(-127, 128, size=(Kd, N)).astype(np.int8)
    s = rng.uniform(0.001, 0.01, size=N).astype(np.float32)
    return to_dev(a), to_dev(wq), to_dev(s)


def _att_case(seed, B=1, H=2, Sq=64, Skv=4096, D=128):
    return tuple(to_dev(rng_bf16(shape, seed + i))
                 for i, shape in enumerate([(B, H, Sq, D), (B, H, Skv, D), (B, H, Skv, D)]))


def _run_thread(fn, iters, results, idx, errors, stream):
    import torch

    try:
        with torch.cuda.stream(stream):
            outs = [fn(i) for i in range(iters)]
        stream.synchronize()
        results[idx] = [from_dev(o) for o in outs]
    except Exception as e:  # noqa: BLE001 -- re-raised in the main thread
        errors.append(e)


def test_split_workspaces_concurrent_streams(gpu):
    import torch

    from polykernel_amd import kernels, runtime as rt

    cfg = rt.default_config("matmul_int8", 16, 4096, 8192)
    assert cfg["block_k"] < 8192, f"expected a split-K plan, got {cfg}"
    i8 = [_int8_case(10 + j) for j in range(3)]
    att = [_att_case(20 + 3 * j) for j in range(3)]
    scale = 1.0 / np.sqrt(128)
    run_i8 = lambda i: kernels.matmul_int8(*i8[i % 3])
    run_att = lambda i: kernels.attention_prefill(*att[i % 3], scale=scale, causal=True)
    _say("serial reference runs")
    want_i8 = [from_dev(kernels.matmul_int8(*c)) for c in i8]
    want_att = [from_dev(kernels.attention_prefill(*c, scale=scale, causal=True)) for c in att]
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    results, errors = [None, None], []
    iters = 24
    t1 = threading.Thread(target=_run_thread, args=(run_i8, iters, results, 0, errors, s1))
    t2 = threading.Thread(target=_run_thread, args=(run_att, iters, results, 1, errors, s2))
    _say("concurrent: int8 split-K on stream 1, attention split-KV on stream 2")
    t1.start(), t2.start()
    t1.join(120), t2.join(120)
    assert not errors, errors
    assert not t1.is_alive() and not t2.is_alive()
    for i in range(iters):
        assert np.array_equal(results[0][i], want_i8[i % 3]), f"int8 launch {i} differs from the serial run"
        assert np.array_equal(results[1][i], want_att[i % 3]), f"attention launch {i} differs from the serial run"


def test_split_workspace_one_stream_two_threads(gpu):
    """Two threads feeding ONE stream: each split-K launch's partial-sum and
    reduction kernels stay adjacent in the stream (the workspace slot's lock
    is held while they are enqueued)."""
    import torch

    from polykernel_amd import kernels

    cases = [_int8_case(40 + j) for j in range(4)]
    want = [from_dev(kernels.matmul_int8(*c)) for c in cases]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    results, errors = [None, None], []
    iters = 32
    t1 = threading.Thread(target=_run_thread,
                          args=(lambda i: kernels.matmul_int8(*cases[i % 2]), iters, results, 0, errors, s))
    t2 = threading.Thread(target=_run_thread,
                          args=(lambda i: kernels.matmul_int8(*cases[2 + i % 2]), iters, results, 1, errors, s))
    t1.start(), t2.start()
    t1.join(120), t2.join(120)
    assert not errors, errors
    for i in range(iters):
        assert np.array_equal(results[0][i], want[i % 2])
        assert np.array_equal(results[1][i], want[2 + i % 2])


def test_dma_gemm_a_operand_beyond_4gib(gpu, oracle):
    """M = 262656, K = 8192: A is 4.3 GB (> 2^32 bytes).  Tile row 512 starts
    where (M - m0) K 2 is exactly 2^32, the row block a whole-matrix record
    count would have truncated to zero length."""
    import torch

    M, Kd, N = 262656, 8192, 256
    assert M * Kd * 2 > 2**32
    _say(f"matmul {M}x{N}x{Kd} (A {M * Kd * 2 / 2**30:.2f} GiB), integer inputs")
    gen = torch.Generator(device="cuda").manual_seed(7)
    A = torch.empty((M, Kd), dtype=torch.bfloat16, device="cuda")
    for r0 in range(0, M, 8192):
        r1 = min(M, r0 + 8192)
        A[r0:r1] = torch.randint(-3, 4, (r1 - r0, Kd), device="cuda", generator=gen).to(torch.bfloat16)
    b = int_bf16((Kd, N), 8)
    from polykernel_amd import kernels

    C = kernels.matmul(A, to_dev(b))
    torch.cuda.synchronize()
    rows = np.concatenate([np.arange(0, 4), np.arange(508, 516), np.arange(764, 772),
                           np.arange(M - 262144 - 4, M - 262144 + 4), np.arange(M - 8, M),
                           np.random.default_rng(9).choice(M, 16, replace=False)])
    rows = np.unique(rows)
    idx = torch.from_numpy(rows).cuda()
    a_rows = from_dev(A.index_select(0, idx).contiguous())
    got = from_dev(C.index_select(0, idx).contiguous())
    want = oracle.matmul(a_rows, b)
    bad = np.flatnonzero((got != want).any(axis=1))
    assert bad.size == 0, f"rows {rows[bad][:10]} differ"
    del A, C
    torch.cuda.empty_cache()


def test_release_workspace_and_per_thread_stream(gpu):
    """pk_release_workspace frees a stream's library workspace once the
    stream's queued kernels are done: a split-K int8 launch on a new stream,
    the release, the stream dropped, three times over (a new stream may reuse
    the handle), every output equal to the default stream's; releasing a
    stream without a slot is a no-op.  hipStreamPerThread gives each host
    thread its own buffer, and each thread releases its own."""
    import ctypes

    import torch

    from polykernel_amd import _lib, kernels
    from polykernel_amd import runtime as rt

    lib = _lib.load()
    assert rt.default_config("matmul_int8", 16, 4096, 8192)["block_k"] < 8192
    a, wq, s = _int8_case(7)
    want = from_dev(kernels.matmul_int8(a, wq, s))
    for rnd in range(3):
        _say(f"release round {rnd}")
        st = torch.cuda.Stream()
        with torch.cuda.stream(st):
            out = kernels.matmul_int8(a, wq, s)
        _lib.check(lib.pk_release_workspace(st.cuda_stream), "pk_release_workspace")
        assert np.array_equal(from_dev(out), want)
        _lib.check(lib.pk_release_workspace(st.cuda_stream), "pk_release_workspace (no slot)")
        del st, out

    per_thread = 2  # hipStreamPerThread
    ptrs, errors = {}, []
    both = threading.Barrier(2)

    def grab(i):
        try:
            p = ctypes.c_void_p()
            _lib.check(lib.pk_library_workspace(1 << 20, per_thread, ctypes.byref(p)), "pk_library_workspace")
            ptrs[i] = p.value
            both.wait(timeout=60)  # both threads alive: distinct thread ids
            _lib.check(lib.pk_release_workspace(per_thread), "pk_release_workspace")
        except Exception as e:  # noqa: BLE001 -- re-raised in the main thread
            errors.append(e)

    ts = [threading.Thread(target=grab, args=(i,)) for i in range(2)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
    assert not errors, errors
    assert ptrs[0] and ptrs[1] and ptrs[0] != ptrs[1], ptrs


def test_rmsnorm_matmul_panel_in_a_replayed_graph(gpu):
    """The config-1 RMSNorm -> MatMul launch (the whole-K panel kernel, which
    allocates nothing) captured into a HIP graph gives the eager bits on every
    replay, with eager launches and synchronisations between the replays (the
    bench times config 1 and its launch floor this way)."""
    import ctypes

    import torch

    from polykernel_amd import _lib, synth

    lib = _lib.load()
    x = to_dev(synth.normal_bf16((128, 768), 11))
    g = to_dev(synth.normal_bf16((768,), 12, 0.1, 1.0))
    w = to_dev(synth.normal_bf16((768, 3072), 13, 1 / np.sqrt(768)))
    o = torch.empty(128, 3072, dtype=torch.bfloat16, device="cuda")
    eager = torch.empty_like(o)

    def launch(out, sp):
        return lib.launch_fused_rmsnorm_matmul_gamma(x.data_ptr(), g.data_ptr(), w.data_ptr(), out.data_ptr(),
                                                     128, 3072, 768, ctypes.c_float(1e-6), sp)

    assert launch(eager, torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        assert launch(o, s.cuda_stream) == 0
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=s):
            sp = torch.cuda.current_stream().cuda_stream
            for _ in range(4):
                assert launch(o, sp) == 0
    for rep in range(5):
        o.fill_(0)
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        _say(f"graph replay {rep}")
        assert torch.equal(o.view(torch.int16), eager.view(torch.int16)), rep
        assert launch(eager, torch.cuda.current_stream().cuda_stream) == 0  # eager work between replays
        torch.cuda.synchronize()


def test_mlp_block_and_decode_chain_in_replayed_graphs(gpu):
    """The two block entry points with caller workspace (launch_mlp_block: RMSNorm
    + two DMA GEMMs; launch_decode_mlp_int8: two split-K int8 streams + their
    reductions) allocate and clear nothing, so they can be captured into a HIP
    graph: every replay gives the eager bits, with eager launches and
    synchronisations between the replays."""
    import ctypes

    import torch

    from polykernel_amd import _lib, kernels, synth

    lib = _lib.load()
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731

    M, d, F = 512, 1024, 4096
    x = to_dev(synth.normal_bf16((M, d), 61))
    g = to_dev(synth.normal_bf16((d,), 62, 0.1, 1.0))
    w1 = to_dev(synth.normal_bf16((d, F), 63, 1 / np.sqrt(d)))
    b1 = to_dev(synth.normal_bf16((F,), 64, 0.02))
    w2 = to_dev(synth.normal_bf16((F, d), 65, 1 / np.sqrt(F)))
    b2 = to_dev(synth.normal_bf16((d,), 66, 0.02))
    ws = torch.empty(lib.pk_mlp_block_workspace_size(M, d, F), dtype=torch.uint8, device="cuda")

    def mlp(out, sp):
        return lib.launch_mlp_block(x.data_ptr(), g.data_ptr(), w1.data_ptr(), b1.data_ptr(), w2.data_ptr(),
                                    b2.data_ptr(), out.data_ptr(), M, d, F, ctypes.c_float(1e-6),
                                    ws.data_ptr(), ws.numel(), sp)

    Md, dd, Fd = 16, 4096, 8192
    xq = to_dev(synth.normal_bf16((Md, dd), 67))
    w1q, s1 = kernels.quantize_per_channel(to_dev(synth.normal_bf16((dd, Fd), 68, 1 / np.sqrt(dd))))
    w2q, s2 = kernels.quantize_per_channel(to_dev(synth.normal_bf16((Fd, dd), 69, 1 / np.sqrt(Fd))))
    wsq = torch.empty(lib.pk_decode_mlp_int8_workspace_size(Md, dd, Fd), dtype=torch.uint8, device="cuda")

    def decode(out, sp):
        return lib.launch_decode_mlp_int8(xq.data_ptr(), w1q.data_ptr(), s1.data_ptr(), w2q.data_ptr(),
                                          s2.data_ptr(), out.data_ptr(), Md, dd, Fd, wsq.data_ptr(),
                                          wsq.numel(), sp)

    for name, launch, shape in (("mlp_block", mlp, (M, d)), ("decode_mlp_int8", decode, (Md, dd))):
        o = torch.empty(*shape, dtype=torch.bfloat16, device="cuda")
        eager = torch.empty_like(o)
        assert launch(eager, st()) == 0
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            assert launch(o, s.cuda_stream) == 0
            torch.cuda.synchronize()
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr, stream=s):
                for _ in range(3):
                    assert launch(o, torch.cuda.current_stream().cuda_stream) == 0
        for rep in range(4):
            o.fill_(0)
            torch.cuda.synchronize()
            gr.replay()
            torch.cuda.synchronize()
            _say(f"{name}: graph replay {rep}")
            assert torch.equal(o.view(torch.int16), eager.view(torch.int16)), (name, rep)
            assert launch(eager, st()) == 0  # eager work between replays
            torch.cuda.synchronize()
