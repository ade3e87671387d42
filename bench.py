#!/usr/bin/env python3
"""Benchmark: the config-2 fused MLP block on one MI355X.

    python bench.py [--gpus 1] [--steps 50] [--warmup 40] [--settle-ms 250]

A step is one pass of the MLP block over the config-2 batch (BASELINE.json
configs[1]): RMSNorm(x, gamma) -> MatMul W1 [4096,16384] + b1 -> GELU(erf) ->
MatMul W2 [16384,4096] + b2 -> + x, x bf16 [4096,4096], synthetic seeded inputs
resident in HBM before timing.  The step issues the same three launches
launch_mlp_block makes (rmsnorm, GEMM+bias+GELU, GEMM+bias+residual); the two
GEMMs are served by the runtime (detect -> select -> serve) from the committed
gfx950 tuning cache (polykernel_amd/tuning/gfx950.json, written by the
correctness-gated autotuner), with HIP events around the dominant GEMM launch
on the stream it runs on.

value = 2^40 algorithmic FLOP per step / wall time per step (TFLOP/s), over
exactly --steps timed steps after --warmup untimed ones, which follow
--settle-ms of untimed steps (the clocks climb for ~50 steps after the idle
input set-up).
The other BASELINE configs (attention prefill, residual+RMSNorm, masked
softmax, int8 decode, RMSNorm->MatMul) are reported under "extra", each with
the CPU oracle timed on one thread and on all threads (a bounded sample,
extrapolated per row / head where it is smaller than the workload, repeated
until ~10 s of CPU time per leg) and the
parity of the GPU output on that sample; the config-2 oracle timing is
"cpu_baseline".  One JSON line is printed.

    python bench.py --only cfg4a [--no-cpu]   # one config (for rocprofv3 runs)
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "fused-MLP TFLOP/s (% bf16 MFMA peak); attn-prefill TFLOP/s; GB/s; 1×MI355X"
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
SEED = 0xC0FFEE

M, D, F = 4096, 4096, 16384
MLP_FLOP = 2 * M * D * F * 2           # 2^40
GEMM_FLOP = 2 * M * D * F              # per GEMM launch


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def dev_bf16(a):
    import numpy as np
    import torch

    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def event_pair(fence: bool = False):
    """Two timing events: TimingEvent (no cache maintenance at record) unless
    `fence`, for timings that must start from written-back caches (the
    MALL-flushed launches)."""
    import torch

    if fence:
        return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    return TimingEvent(), TimingEvent()


class TimingEvent:
    """A HIP event created with hipEventDisableSystemFence (0x20000000), for the
    per-step kernel timing inside the timed region: recording a default event
    also performs a system-scope cache write-back and invalidate, which timing
    needs no part of and which slows the work around it (measured on MI355X:
    four default events per MLP step added 14 us to the 0.885 ms step, four
    of these 7 us).  Same HIP runtime as torch's streams: the libamdhip64 that
    torch loaded."""

    _hip = None

    @classmethod
    def _lib(cls):
        if cls._hip is None:
            import ctypes as C

            paths = sorted({ln.split()[-1] for ln in open("/proc/self/maps") if "libamdhip64" in ln})
            if not paths:
                raise RuntimeError("libamdhip64 is not loaded (initialise torch's HIP first)")
            hip = C.CDLL(paths[0])
            hip.hipEventCreateWithFlags.argtypes = [C.POINTER(C.c_void_p), C.c_uint]
            hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
            hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
            hip.hipEventDestroy.argtypes = [C.c_void_p]
            cls._hip = hip
        return cls._hip

    def __init__(self):
        import ctypes as C

        self.h = C.c_void_p()
        rc = self._lib().hipEventCreateWithFlags(C.byref(self.h), 0x20000000)
        if rc != 0:
            raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")

    def record(self, stream=None) -> None:
        import ctypes as C

        import torch

        st = (stream or torch.cuda.current_stream()).cuda_stream
        rc = self._lib().hipEventRecord(self.h, C.c_void_p(st))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def elapsed_time(self, end: "TimingEvent") -> float:
        """ms from this event to `end` (both recorded and complete)."""
        import ctypes as C

        ms = C.c_float()
        rc = self._lib().hipEventElapsedTime(C.byref(ms), self.h, end.h)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return ms.value

    def __del__(self):
        if self._hip is not None and self.h:
            self._hip.hipEventDestroy(self.h)


def bench_mlp(steps: int, warmup: int, settle_ms: float = 250.0):
    import numpy as np
    import torch

    from polykernel_amd import _lib, synth
    from polykernel_amd._lib import check

    from polykernel_amd import runtime as prt

    lib = _lib.load()
    served = prt.default_runtime()
    entry1 = served.resolve("fused_matmul_bias_gelu", M, F, D)
    entry2 = served.resolve("fused_matmul_bias_residual", M, D, F)
    log(f"served configs: gemm1 {entry1['best']}, gemm2 {entry2['best']}")
    t0 = time.time()
    x = synth.normal_bf16((M, D), 1, seed=SEED)
    g = synth.normal_bf16((D,), 2, 0.1, 1.0, seed=SEED)
    w1 = synth.normal_bf16((D, F), 3, 1.0 / math.sqrt(D), seed=SEED)
    b1 = synth.normal_bf16((F,), 4, 0.02, seed=SEED)
    w2 = synth.normal_bf16((F, D), 5, 1.0 / math.sqrt(F), seed=SEED)
    b2 = synth.normal_bf16((D,), 6, 0.02, seed=SEED)
    tx, tg, tw1, tb1, tw2, tb2 = map(dev_bf16, (x, g, w1, b1, w2, b2))
    a = torch.empty(M, D, dtype=torch.bfloat16, device="cuda")
    h = torch.empty(M, F, dtype=torch.bfloat16, device="cuda")
    y = torch.empty(M, D, dtype=torch.bfloat16, device="cuda")
    log(f"mlp inputs ready in {time.time() - t0:.1f}s")
    stream = torch.cuda.current_stream()
    sp = stream.cuda_stream

    io1 = prt.MatmulIO(A=a.data_ptr(), B=tw1.data_ptr(), C=h.data_ptr(), bias=tb1.data_ptr(), residual=None,
                       M=M, N=F, K=D, stream=sp)
    io2 = prt.MatmulIO(A=h.data_ptr(), B=tw2.data_ptr(), C=y.data_ptr(), bias=tb2.data_ptr(),
                       residual=tx.data_ptr(), M=M, N=D, K=F, stream=sp)

    # ev1: events around GEMM1 (the timed steps: the roofline kernel's duration);
    # ev2: around GEMM2 (extra steps after the timed ones, for the breakdown)
    def step(ev1=None, ev2=None):
        check(lib.launch_rmsnorm(tx.data_ptr(), tg.data_ptr(), a.data_ptr(), M, D, 1e-6, sp), "rmsnorm")
        if ev1 is not None:
            ev1[0].record(stream)
        served.run("fused_matmul_bias_gelu", M, F, D, io1)
        if ev1 is not None:
            ev1[1].record(stream)
        if ev2 is not None:
            ev2[0].record(stream)
        served.run("fused_matmul_bias_residual", M, D, F, io2)
        if ev2 is not None:
            ev2[1].record(stream)

    # Clock settle before the warmup steps: untimed steps for settle_ms of wall
    # time.  After the idle input set-up the first ~50 steps run ~5-10 % slow
    # while the clocks climb to their sustained state (0.98 ms per step measured
    # with 5 warmups, 0.89-0.92 ms after 40 or more), so with few warmup steps the
    # timed steps would sample that ramp rather than the block's sustained rate.
    settle_steps = 0
    t_end = time.perf_counter() + settle_ms * 1e-3
    while time.perf_counter() < t_end:
        for _ in range(8):
            step()
        settle_steps += 8
        torch.cuda.synchronize()
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    log(f"clock settle: {settle_steps} untimed steps in {settle_ms:.0f} ms, then {warmup} warmup steps")
    evs = [[TimingEvent(), TimingEvent()] for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(ev1=evs[i])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    # GEMM2 for the breakdown: 10 more steps at once, while the clocks are in the
    # sustained state (after an idle spell the first steps run slow)
    evs2 = [[TimingEvent(), TimingEvent()] for _ in range(10)]
    for i in range(10):
        step(ev2=evs2[i])
    torch.cuda.synchronize()
    g1 = [e[0].elapsed_time(e[1]) for e in evs]
    g2 = [e[0].elapsed_time(e[1]) for e in evs2]
    y_host = from_dev_bits(y)  # the served path's output (the same bits every step), for the parity sample

    # the library's plain entry point (its built-in configs) on the same
    # buffers: equal work, reported beside the served path
    ws = torch.empty(lib.pk_mlp_block_workspace_size(M, D, F), dtype=torch.uint8, device="cuda")
    def entry():
        check(lib.launch_mlp_block(tx.data_ptr(), tg.data_ptr(), tw1.data_ptr(), tb1.data_ptr(),
                                   tw2.data_ptr(), tb2.data_ptr(), y.data_ptr(), M, D, F, 1e-6,
                                   ws.data_ptr(), ws.numel(), sp), "launch_mlp_block")

    for _ in range(20):  # back to the sustained clocks after the host copy above
        entry()
    e0, e1 = event_pair()
    e0.record(stream)
    for _ in range(5):
        entry()
    e1.record(stream)
    torch.cuda.synchronize()
    entry_ms = e0.elapsed_time(e1) / 5
    inputs = dict(x=x, g=g, w1=w1, b1=b1, w2=w2, b2=b2, y_gpu=y_host,
                  entry_equal=bool(np.array_equal(from_dev_bits(y), y_host)))
    return elapsed, g1, g2, entry_ms, inputs, (entry1, entry2), settle_steps


class Timer:
    """HIP-event timing on torch's current stream (the stream every launch
    below is issued on)."""

    def __init__(self, reps: int = 20):
        import torch

        self.reps = reps
        self.stream = torch.cuda.current_stream()
        self.sp = self.stream.cuda_stream
        self.stats = {}

    def __call__(self, fn, key=None, warm=3, flush=None, warm_s=0.05):
        """Mean per launch over `reps` back-to-back launches (the median of
        three such batches; per-launch pairs of events when `flush` runs
        between launches); with `key`, the median and minimum of `reps`
        launches timed one by one go into stats[key].

        Before timing, `warm` launches and then `warm_s` seconds of sustained
        launches: the memory and fabric clocks fall within milliseconds of
        idle and take ~15 ms of load to climb back (measured: the first 20-launch
        batches of config 4a after setup ran 131-143 us per launch, later ones
        124-126 us), and production code runs these kernels back to back."""
        import torch

        n, stream = self.reps, self.stream
        for _ in range(warm):
            fn()
        if warm_s > 0 and flush is None:
            e0, e1 = event_pair()
            e0.record(stream)
            fn()
            e1.record(stream)
            torch.cuda.synchronize()
            per_s = max(e0.elapsed_time(e1) * 1e-3, 1e-6)
            for _ in range(min(int(warm_s / per_s) + 1, 20000)):
                fn()
        evs = [event_pair(fence=flush is not None) for _ in range(n)]
        for e0, e1 in evs:
            if flush is not None:
                flush()
            e0.record(stream)
            fn()
            e1.record(stream)
        torch.cuda.synchronize()
        t = sorted(e0.elapsed_time(e1) for e0, e1 in evs)
        if key:
            self.stats[key] = {"median_us": round(t[n // 2] * 1e3, 2), "min_us": round(t[0] * 1e3, 2)}
        if flush is not None:
            return sum(t) / n
        # three batches of n back-to-back launches, the median batch mean: per-launch
        # times drift by ~10 % over a few ms within one process (clocks, power)
        means = []
        for _ in range(3):
            e0, e1 = event_pair()
            e0.record(stream)
            for _ in range(n):
                fn()
            e1.record(stream)
            torch.cuda.synchronize()
            means.append(e0.elapsed_time(e1) / n)
        return sorted(means)[1]


def graph_time(launch, n: int = 100, reps: int = 20) -> float:
    """ms per launch of launch(stream) captured n times in a HIP graph on a side
    stream and replayed `reps` times (median): the GPU time of back-to-back
    launches without the host's per-launch cost.  launch must not allocate or
    set memory (nothing to capture but kernels)."""
    import torch

    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        assert launch(s.cuda_stream) == 0
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr, stream=s):
            sp = torch.cuda.current_stream().cuda_stream
            for _ in range(n):
                assert launch(sp) == 0
    for _ in range(5):
        gr.replay()
    torch.cuda.synchronize()
    t = []
    for _ in range(reps):
        e0, e1 = event_pair()
        e0.record()
        gr.replay()
        e1.record()
        torch.cuda.synchronize()
        t.append(e0.elapsed_time(e1) / n)
    return sorted(t)[reps // 2]


def host_info() -> dict:
    """The host the CPU baselines ran on: usable cores and CPU model."""
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count()
    return {"nproc": usable, "cpu_model": model}


CPU_LEG_SECONDS = 10.0  # CPU work per baseline leg: the sample is run again until this much time has passed


def cpu_pair(run, single_sample, all_sample, unit: str, work_per_unit: float, total_units: float,
             what: str, leg_seconds: float = CPU_LEG_SECONDS) -> dict:
    """Time the oracle (the C restatement of kernels/cpu) on one thread and on
    every thread OpenMP gives it: run(sample) processes `sample` units (rows,
    queries, ...) of the workload, `work_per_unit` is the metric's work (FLOP
    or algorithmic bytes) per unit, extrapolated to `total_units` when the
    sample is smaller than the workload.  Each leg repeats its sample until
    `leg_seconds` of CPU time have passed (at least once)."""
    from oracle import pyoracle

    threads = pyoracle.num_threads()
    res = {}
    for name, sample, nthr in (("single_thread", single_sample, 1), ("all_cores", all_sample, threads)):
        pyoracle.set_num_threads(nthr)
        try:
            t0 = time.perf_counter()
            out = run(sample)
            reps = 1
            while time.perf_counter() - t0 < leg_seconds:
                run(sample)
                reps += 1
            dt = time.perf_counter() - t0
        finally:
            pyoracle.set_num_threads(threads)
        scale = 1e12 if unit == "TFLOP/s" else 1e9
        res[name] = {"value": round(reps * sample * work_per_unit / dt / scale, 6), "unit": unit, "cores": nthr,
                     "kind": "port", "seconds": round(dt, 3), "repetitions": reps,
                     "sample": f"{sample:g} of {total_units:g} {what}" +
                               (" (extrapolated per unit)" if sample < total_units else " (full workload)") +
                               f", run {reps} times"}
        res.setdefault("_outputs", {})[name] = out
    return res


def _parity(got_bits, want_bits) -> dict:
    from polykernel_amd import metrics

    rep = metrics.report(got_bits, want_bits)
    return {"cosine": round(rep.cosine, 7), "pcc": round(rep.pcc, 7), "max_rel_err": float(f"{rep.max_rel_err:.3e}"),
            "bit_exact": round(rep.bit_exact, 6), "max_ulp": rep.max_ulp}


def _finish_cpu(entry: dict, cpu: dict, gpu_bits, ref_of) -> None:
    """Attach the CPU timings and the parity of the GPU output on the oracle's
    all-cores sample (ref_of maps the oracle output onto the GPU slice)."""
    outs = cpu.pop("_outputs")
    entry["cpu_baseline"] = cpu
    want, got = ref_of(outs["all_cores"], gpu_bits)
    entry["parity_sample"] = _parity(got, want)


def from_dev_bits(t):
    import numpy as np
    import torch

    t = t.detach().cpu()
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()


CFG1_BYTES = 5703168   # x 196,608 + gamma 1,536 + W 4,718,592 + out 786,432


def bench_cfg1(t: Timer, cpu: bool) -> dict:
    """Config 1: RMSNorm -> MatMul fragment (cache-resident), warm and cold."""
    import torch

    from polykernel_amd import _lib, synth
    from polykernel_amd._lib import check

    lib = _lib.load()
    hx = synth.normal_bf16((128, 768), 11)
    hg = synth.normal_bf16((768,), 12, 0.1, 1.0)
    hw = synth.normal_bf16((768, 3072), 13, 1 / math.sqrt(768))
    x, g, w = dev_bf16(hx), dev_bf16(hg), dev_bf16(hw)
    o = torch.empty(128, 3072, dtype=torch.bfloat16, device="cuda")
    run = lambda: check(lib.launch_fused_rmsnorm_matmul_gamma(
        x.data_ptr(), g.data_ptr(), w.data_ptr(), o.data_ptr(), 128, 3072, 768, 1e-6, t.sp), "cfg1")
    ms = t(run, key="warm")
    big = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    ms_cold = t(run, key="cold", flush=lambda: big.fill_(1))
    # the fixed cost of a launch of the panel kernel's geometry (192 workgroups
    # of 256 threads, 144 KiB of dynamic LDS): launched from this loop the empty
    # kernel is bound by the host's launch rate, so its GPU-side cost comes from
    # a replayed HIP graph of 100 launches, and config 1 is timed that way too
    tiles, lds = (128 // 32) * (3072 // 64), 768 * 128 + 32 * 768 * 2
    floor = lambda: check(lib.pk_probe_empty_launch(tiles, 256, lds, t.sp), "empty launch")
    ms_floor_eager = t(floor, key="floor")
    want = o.clone()
    ms_graph = graph_time(lambda sp: lib.launch_fused_rmsnorm_matmul_gamma(
        x.data_ptr(), g.data_ptr(), w.data_ptr(), o.data_ptr(), 128, 3072, 768, 1e-6, sp))
    graph_equal = bool(torch.equal(o.view(torch.int16), want.view(torch.int16)))
    ms_floor = graph_time(lambda sp: lib.pk_probe_empty_launch(tiles, 256, lds, sp))
    flop = 2 * 128 * 3072 * 768
    roof_us = CFG1_BYTES / (PEAK_HBM_GBS * 1e9) * 1e6

    def roof(ms_):
        gbs = CFG1_BYTES / (ms_ * 1e-3) / 1e9
        return {"achieved": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4)}

    out = {"us": round(ms * 1e3, 2), "tflops": round(flop / (ms * 1e-3) / 1e12, 2),
           "warm": t.stats["warm"], "cold_us": round(ms_cold * 1e3, 2), "cold": t.stats["cold"],
           "roofline": {"bound": "hbm", "unit": "GB/s", "peak": PEAK_HBM_GBS, "bytes": CFG1_BYTES,
                        "time_at_peak_us": round(roof_us, 3), "warm": roof(ms), "cold": roof(ms_cold),
                        "graph": roof(ms_graph),
                        "mfma_time_at_peak_us": round(flop / (PEAK_BF16_TFLOPS * 1e12) * 1e6, 3)},
           "graph_us": round(ms_graph * 1e3, 2), "graph_output_equal": graph_equal,
           "launch_floor_us": round(ms_floor * 1e3, 2), "launch_floor_eager_us": round(ms_floor_eager * 1e3, 2),
           "note": "warm: L2/MALL-resident (5.7 MB), launched back to back; cold: a 1 GiB buffer written between "
                   "launches; graph_us: per launch in a replayed HIP graph of 100 launches (GPU time, no host "
                   "launch cost); launch_floor_us: an empty kernel with the panel kernel's grid, workgroup and "
                   "LDS in such a graph (launch_floor_eager_us: the same launched from the loop, host-bound)"}
    del big
    if cpu:
        from oracle import pyoracle

        c = cpu_pair(lambda n: pyoracle.fused_rmsnorm_matmul(hx, hw, hg, 1e-6), 128, 128, "TFLOP/s",
                     flop / 128, 128, "rows of x [128,768] @ W [768,3072]")
        _finish_cpu(out, c, from_dev_bits(o), lambda want, got: (want, got))
    return out


def _cfg3_inputs():
    from polykernel_amd import synth

    B, H, Sc, Sn, Dh = 1, 32, 3584, 512, 128
    return dict(B=B, H=H, Sc=Sc, Sn=Sn, Dh=Dh,
                q=synth.normal_bf16((B, H, Sn, Dh), 21), kn=synth.normal_bf16((B, H, Sn, Dh), 22),
                vn=synth.normal_bf16((B, H, Sn, Dh), 23), kc=synth.normal_bf16((B, H, Sc, Dh), 24),
                vc=synth.normal_bf16((B, H, Sc, Dh), 25))


CFG3_FLOP = 32216449024   # 4 * D per unmasked (query, key) pair


def bench_cfg3(t: Timer, cpu: bool) -> dict:
    """Config 3: KV append (in place) + causal prefill, B1 H32 D128, 3584 + 512."""
    import numpy as np
    import torch

    from polykernel_amd import _lib
    from polykernel_amd._lib import check

    lib = _lib.load()
    h = _cfg3_inputs()
    B, H, Sc, Sn, Dh = h["B"], h["H"], h["Sc"], h["Sn"], h["Dh"]
    scale = 1 / math.sqrt(Dh)
    q, kn, vn = dev_bf16(h["q"]), dev_bf16(h["kn"]), dev_bf16(h["vn"])
    kc = torch.empty(B, H, Sc + Sn, Dh, dtype=torch.bfloat16, device="cuda")
    vc = torch.empty_like(kc)
    kc[:, :, :Sc] = dev_bf16(h["kc"])
    vc[:, :, :Sc] = dev_bf16(h["vc"])
    o = torch.empty_like(q)
    run = lambda: check(lib.launch_fused_kv_append_attention(
        q.data_ptr(), kc.data_ptr(), vc.data_ptr(), kn.data_ptr(), vn.data_ptr(), o.data_ptr(),
        B, H, Sn, Sc, Dh, Sc + Sn, scale, 1, t.sp), "cfg3")
    ms = t(run, key="cfg3")
    big = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    ms_cold = t(run, key="cfg3_cold", flush=lambda: big.fill_(1))
    del big
    tf = CFG3_FLOP / (ms * 1e-3) / 1e12
    tf_cold = CFG3_FLOP / (ms_cold * 1e-3) / 1e12
    out = {"us": round(ms * 1e3, 2), "tflops": round(tf, 2), "frac_mfma": round(tf / PEAK_BF16_TFLOPS, 4),
           **t.stats["cfg3"],
           "cold_us": round(ms_cold * 1e3, 2), "tflops_cold": round(tf_cold, 2),
           "frac_mfma_cold": round(tf_cold / PEAK_BF16_TFLOPS, 4), "cold": t.stats["cfg3_cold"],
           "note": "us/tflops: back-to-back launches, the 84 MB of Q/K/V/O stay resident in the 256 MB MALL "
                   "(cache-resident); cold: a 1 GiB buffer written before each launch (MALL flushed)"}
    if cpu:
        from oracle import pyoracle

        kfull = np.concatenate([h["kc"], h["kn"]], axis=2)
        vfull = np.concatenate([h["vc"], h["vn"]], axis=2)
        # heads are independent and equal work: time whole heads
        run = lambda nh: pyoracle.attention_prefill(h["q"][:, :nh], kfull[:, :nh], vfull[:, :nh], scale, True)
        c = cpu_pair(run, 1, 16, "TFLOP/s", CFG3_FLOP / H, H, "heads (all 512 queries, 4096 keys each)")
        _finish_cpu(out, c, from_dev_bits(o), lambda want, got: (want, got[:, :want.shape[1]]))
    return out


def bench_cfg4a(t: Timer, cpu: bool) -> dict:
    """Config 4a: residual + RMSNorm [16384, 8192]."""
    import torch

    from polykernel_amd import _lib, synth
    from polykernel_amd._lib import check

    lib = _lib.load()
    R, C = 16384, 8192
    hx, hr = synth.normal_bf16((R, C), 31), synth.normal_bf16((R, C), 32)
    hg = synth.normal_bf16((C,), 33, 0.1, 1.0)
    xa, ra, ga = dev_bf16(hx), dev_bf16(hr), dev_bf16(hg)
    oa = torch.empty_like(xa)
    ms = t(lambda: check(lib.launch_fused_residual_rmsnorm(
        xa.data_ptr(), ra.data_ptr(), ga.data_ptr(), oa.data_ptr(), R, C, 1e-6, t.sp), "cfg4a"), key="cfg4a")
    nbytes = 805322752
    gbs = nbytes / (ms * 1e-3) / 1e9
    out = {"us": round(ms * 1e3, 2), "gbs": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
           **t.stats["cfg4a"]}
    if cpu:
        from oracle import pyoracle

        run = lambda n: pyoracle.residual_rmsnorm(hx[:n], hr[:n], hg, 1e-6)
        c = cpu_pair(run, 2048, R, "GB/s", nbytes / R, R, "rows of [16384,8192]")
        _finish_cpu(out, c, from_dev_bits(oa), lambda want, got: (want, got))
    return out


def bench_cfg4b(t: Timer, cpu: bool) -> dict:
    """Config 4b: masked softmax, fp32 logits [16384, 8192] + bf16 additive mask."""
    import torch

    from polykernel_amd import _lib, synth
    from polykernel_amd._lib import check

    lib = _lib.load()
    R, C = 16384, 8192
    hl, hm = synth.normal_f32((R, C), 34, 2.0), synth.mask_bf16((R, C), 35, 0.1)
    lg, mk = torch.from_numpy(hl).cuda(), dev_bf16(hm)
    om = torch.empty(R, C, dtype=torch.bfloat16, device="cuda")
    ms = t(lambda: check(lib.launch_fused_softmax_mask(lg.data_ptr(), mk.data_ptr(), om.data_ptr(), R, C, t.sp),
                         "cfg4b"), key="cfg4b")
    nbytes = 1073741824
    gbs = nbytes / (ms * 1e-3) / 1e9
    out = {"us": round(ms * 1e3, 2), "gbs": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
           **t.stats["cfg4b"]}
    if cpu:
        from oracle import pyoracle

        run = lambda n: pyoracle.softmax_mask(hl[:n], hm[:n])
        c = cpu_pair(run, 1024, R, "GB/s", nbytes / R, R, "rows of [16384,8192]")
        _finish_cpu(out, c, from_dev_bits(om), lambda want, got: (want, got))
    return out


CFG5_BYTES = 470433792


def bench_cfg5(t: Timer, cpu: bool) -> dict:
    """Config 5: int8 decode MLP, M=16, 8192 <-> 28672 (weights quantised on the
    GPU); the runtime-served tuned configs over two weight copies used in turn,
    and the library's launch_decode_mlp_int8 beside it."""
    import torch

    from polykernel_amd import _lib, kernels, synth
    from polykernel_amd import runtime as prt
    from polykernel_amd._lib import check

    lib = _lib.load()
    sp = t.sp
    Md, dd, Fd = 16, 8192, 28672
    hx = synth.normal_bf16((Md, dd), 41)
    xd = dev_bf16(hx)
    w1q, s1 = kernels.quantize_per_channel(dev_bf16(synth.normal_bf16((dd, Fd), 42, 1 / math.sqrt(dd))))
    w2q, s2 = kernels.quantize_per_channel(dev_bf16(synth.normal_bf16((Fd, dd), 43, 1 / math.sqrt(Fd))))
    torch.cuda.empty_cache()
    ws = torch.empty(lib.pk_decode_mlp_int8_workspace_size(Md, dd, Fd), dtype=torch.uint8, device="cuda")
    od = torch.empty_like(xd)
    # two copies of the weights, used in turn: 940 MB, so the 256 MB MALL
    # holds none of a call's weights when it starts
    wsets = [(w1q, w2q), (w1q.clone(), w2q.clone())]
    turn = [0]

    def decode():
        a, b = wsets[turn[0] % 2]
        turn[0] += 1
        check(lib.launch_decode_mlp_int8(
            xd.data_ptr(), a.data_ptr(), s1.data_ptr(), b.data_ptr(), s2.data_ptr(), od.data_ptr(),
            Md, dd, Fd, ws.data_ptr(), ws.numel(), sp), "cfg5")

    ms_entry = t(decode)
    served = prt.default_runtime()
    hd = torch.empty(Md, Fd, dtype=torch.bfloat16, device="cuda")
    ios = []
    for a, b in wsets:
        ios.append((prt.MatmulInt8IO(A=xd.data_ptr(), Wq=a.data_ptr(), scale=s1.data_ptr(), C=hd.data_ptr(),
                                     residual=None, M=Md, N=Fd, K=dd, workspace=None, workspace_bytes=0,
                                     stream=sp),
                    prt.MatmulInt8IO(A=hd.data_ptr(), Wq=b.data_ptr(), scale=s2.data_ptr(), C=od.data_ptr(),
                                     residual=xd.data_ptr(), M=Md, N=dd, K=Fd, workspace=None,
                                     workspace_bytes=0, stream=sp)))

    def decode_served():
        i1, i2 = ios[turn[0] % 2]
        turn[0] += 1
        served.run("matmul_int8_gelu", Md, Fd, dd, i1)
        served.run("matmul_int8_residual", Md, dd, Fd, i2)

    ms = t(decode_served, key="cfg5")
    gbs = CFG5_BYTES / (ms * 1e-3) / 1e9
    out = {"us": round(ms * 1e3, 2), "gbs": round(gbs, 1), "frac_hbm": round(gbs / PEAK_HBM_GBS, 4),
           **t.stats["cfg5"], "launch_decode_mlp_int8_us": round(ms_entry * 1e3, 2),
           "served_configs": [served.resolve("matmul_int8_gelu", Md, Fd, dd)["best"],
                              served.resolve("matmul_int8_residual", Md, dd, Fd)["best"]],
           "note": "runtime-served tuned configs; 2 weight copies in turn (no MALL reuse)"}
    if cpu:
        from oracle import pyoracle

        torch.cuda.synchronize()
        hw1, hs1, hw2, hs2 = (from_dev_bits(v) for v in (w1q, s1, w2q, s2))
        run = lambda n: pyoracle.decode_mlp_int8(hx[:n], hw1, hs1, hw2, hs2)
        # rows of x are independent: each row streams every weight once
        c = cpu_pair(run, 1, Md, "GB/s", CFG5_BYTES / Md, Md, "rows of x [16,8192] through W1 and W2")
        _finish_cpu(out, c, from_dev_bits(od), lambda want, got: (want, got))
    return out


EXTRA = {"cfg1": ("rmsnorm_matmul_cfg1", bench_cfg1), "cfg3": ("attention_prefill_cfg3", bench_cfg3),
         "cfg4a": ("residual_rmsnorm_cfg4a", bench_cfg4a), "cfg4b": ("masked_softmax_cfg4b", bench_cfg4b),
         "cfg5": ("int8_decode_mlp_cfg5", bench_cfg5)}


def bench_extra(cpu: bool, only=None, reps: int = 20) -> dict:
    """The other BASELINE configs: GPU time per launch (Timer), and with `cpu`
    the oracle on one thread and on all threads plus the parity of the GPU
    output on the oracle's sample."""
    import torch

    out = {}
    for name, (key, fn) in EXTRA.items():
        if only and name != only:
            continue
        out[key] = fn(Timer(reps), cpu)
        torch.cuda.empty_cache()
    return out


def cpu_baseline(inputs, budget_s: float = 12.0):
    """Oracle (C port of kernels/cpu) on a row sample of the same workload."""
    import numpy as np

    from oracle import pyoracle

    lib = pyoracle.lib()
    threads = pyoracle.num_threads()
    x = inputs["x"]
    rows = 16
    t0 = time.perf_counter()
    outs = [pyoracle.mlp_block(x[:rows], inputs["g"], inputs["w1"], inputs["b1"], inputs["w2"], inputs["b2"],
                               1e-6)]
    dt = time.perf_counter() - t0
    more = int(max(0, min(M - rows, rows * (budget_s / max(dt, 1e-3) - 1))))
    more = (more // 16) * 16
    if more > 0:
        t1 = time.perf_counter()
        outs.append(pyoracle.mlp_block(x[rows:rows + more], inputs["g"], inputs["w1"], inputs["b1"],
                                       inputs["w2"], inputs["b2"], 1e-6))
        dt += time.perf_counter() - t1
        rows += more
    flop = rows * 2 * (D * F + F * D)
    res = {"value": round(flop / dt / 1e12, 6), "unit": "TFLOP/s", "cores": threads, "kind": "port",
           "sample": f"{rows} of {M} rows of the config-2 MLP block (rows are independent) in "
                     f"{dt:.1f}s; oracle/oracle.c -O2 -ffp-contract=off, OpenMP over rows"}
    return res, np.concatenate(outs, axis=0)


def cpu_baseline_single(inputs, rows: int = 16):
    """The same oracle on one thread (the reference's own CPU path is
    single-threaded): a 16-row sample of config 2, extrapolated per row."""
    from oracle import pyoracle

    threads = pyoracle.num_threads()
    pyoracle.set_num_threads(1)
    try:
        t0 = time.perf_counter()
        pyoracle.mlp_block(inputs["x"][:rows], inputs["g"], inputs["w1"], inputs["b1"], inputs["w2"],
                           inputs["b2"], 1e-6)
        dt = time.perf_counter() - t0
    finally:
        pyoracle.set_num_threads(threads)
    flop = rows * 2 * (D * F + F * D)
    return {"value": round(flop / dt / 1e12, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"{rows} of {M} rows of the config-2 MLP block in {dt:.1f}s, one thread"}


def read_traffic():
    """HBM bytes per GEMM launch from the committed rocprofv3 --pmc summary, if any."""
    p = ROOT / "profiles" / "gemm_bias_gelu_mlp_config2_pmc.txt"
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch="):
            try:
                return int(float(line.split("=", 1)[1]))
            except ValueError:
                return None
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 40 warmup steps: the first ~50 steps after the inputs are built run ~4 % slower
    # while the clocks settle (sustained: 0.89 ms/step over 600 steps)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--settle-ms", type=float, default=250.0,
                    help="untimed MLP steps for this long before the warmup steps (clock settle; 0: none)")
    ap.add_argument("--no-extra", action="store_true", help="skip the other configs")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baselines")
    ap.add_argument("--only", choices=sorted(EXTRA), default=None,
                    help="run only this config (GPU timing; CPU baseline unless --no-cpu) and print its "
                         "results -- the profiling entry point for one kernel family")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only time a 1 GiB device-to-device copy (HBM ceiling and the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: --gpus {args.gpus} is not supported "
              "(the kernels run on one MI355X: token rows, attention heads and int8 weight "
              "columns are the units a multi-GPU run would split)",
              file=sys.stderr, flush=True)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    if args.calibrate_copy:
        n = 1 << 30
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        e0, e1 = event_pair()
        e0.record()
        for _ in range(10):
            dst.copy_(src)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / 10
        print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "ms": round(ms, 4),
                          "gbs_read_plus_write": round(2 * n / (ms * 1e-3) / 1e9, 1)}), flush=True)
        return 0
    from polykernel_amd import _lib

    _lib.load()
    log(f"device: {torch.cuda.get_device_name(0)}")
    if args.only:
        res = bench_extra(cpu=not args.no_cpu, only=args.only)
        print(json.dumps({"only": args.only, "host": host_info(), **res}), flush=True)
        return 0
    elapsed, g1, g2, entry_ms, inputs, entries, settle_steps = bench_mlp(args.steps, args.warmup, args.settle_ms)
    ms_step = elapsed / args.steps * 1e3
    value = MLP_FLOP / (ms_step * 1e-3) / 1e12
    g1_ms = sum(g1) / len(g1)
    g2_ms = sum(g2) / len(g2)
    achieved = GEMM_FLOP / (g1_ms * 1e-3) / 1e12
    log(f"mlp step {ms_step:.3f} ms -> {value:.1f} TFLOP/s; gemm1 {g1_ms:.3f} ms, gemm2 {g2_ms:.3f} ms")
    extra = {"host": host_info()}
    if not args.no_extra:
        extra.update(bench_extra(cpu=not args.no_cpu))
        log(f"extra: {json.dumps(extra)}")
    extra["mlp_block_breakdown"] = {
        "gemm1_bias_gelu_ms": round(g1_ms, 4), "gemm2_bias_residual_ms": round(g2_ms, 4),
        "timing": "gemm1: events around GEMM1 in every timed step; gemm2: events around GEMM2 in 10 "
                  "steps after the timed ones (hipEventDisableSystemFence events)",
        "gemm2_tflops": round(GEMM_FLOP / (g2_ms * 1e-3) / 1e12, 1),
        "launch_mlp_block_ms": round(entry_ms, 4),
        "clock_settle": {"ms": args.settle_ms, "untimed_steps": settle_steps,
                         "note": "untimed steps before the warmup steps, so the timed steps see sustained clocks"},
        "served_configs": [entries[0]["best"], entries[1]["best"]],
        "frac_mfma_block": round(value / PEAK_BF16_TFLOPS, 4)}
    extra["mlp_block_breakdown"]["launch_mlp_block_bits_equal_served"] = inputs["entry_equal"]
    cpu = None
    parity = None
    if not args.no_cpu:
        cpu, want = cpu_baseline(inputs)
        cpu["cpu_model"] = extra["host"]["cpu_model"]
        log(f"cpu baseline: {cpu}")
        parity = {**_parity(inputs["y_gpu"][:want.shape[0]], want),
                  "rows": f"0..{want.shape[0] - 1} of {M} (the cpu_baseline sample)"}
        log(f"parity sample: {parity}")
        extra["cpu_baseline_single_thread"] = cpu_baseline_single(inputs)
        log(f"cpu baseline, one thread: {extra['cpu_baseline_single_thread']}")
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_steps": settle_steps,
        "settle_ms": args.settle_ms,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)/N(0,1/fan_in) bf16, BASELINE config 2)",
        "config": {"workload": "MLP block config2: RMSNorm(x)->x@W1[4096,16384]+b1->GELU(erf)->"
                               "@W2[16384,4096]+b2->+x, x bf16 [4096,4096]",
                   "tokens": M, "d": D, "ffn": F, "flop_per_step": MLP_FLOP},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": read_traffic(),
                     "kernel": f"gemm_dma_kernel<EPI_BIAS_GELU,{entries[0]['best']['shared_memory_stages']},"
                               f"{entries[0]['best']['num_warps']},4> (GEMM1: x@W1+b1->GELU, 2^39 FLOP/launch)"},
        "cpu_baseline": cpu,
        "parity_sample": parity,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
