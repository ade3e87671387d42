"""Write tests/golden/ref_vectors.npz from the reference's own kernels/cpu build.

Run in the container that holds /root/reference after `make -C oracle ref`:

    python tests/golden/make_fixtures.py

Inputs are seeded (numpy PCG64); every output comes from the reference's
compiled kernels/cpu code (oracle/_ref: libpkref.so and the attention /
matmul_quant drivers), never from the restatement being pinned.  The file is
data only (inputs + expected outputs) and lets the oracle be pinned where the
reference tree is absent.
"""
from __future__ import annotations

import sys
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import pyoracle as po  # noqa: E402


def rbf(shape, seed, lo=-1.0, hi=1.0):
    x = np.random.default_rng(seed).uniform(lo, hi, size=shape).astype(np.float32)
    return np.array([po.ref_lib().ref_f32_to_bf16(v) for v in x.reshape(-1)], np.uint16).reshape(shape)


def main() -> None:
    if not po.ref_available():
        raise SystemExit("build the reference first: make -C oracle ref")
    ref = po.ref_lib()
    z = {}
    # rmsnorm with gamma
    x, w = rbf((5, 96), 1), rbf((96,), 2, 0.5, 1.5)
    out = np.empty_like(x)
    ref.ref_rmsnorm(x.ctypes.data, w.ctypes.data, out.ctypes.data, 5, 96, np.float32(1e-6))
    z.update(rms_x=x, rms_w=w, rms_eps=np.float32(1e-6), rms_out=out)
    # matmul, odd shape
    a, b = rbf((13, 37), 3), rbf((37, 11), 4)
    out = np.empty((13, 11), np.uint16)
    ref.ref_matmul(a.ctypes.data, b.ctypes.data, out.ctypes.data, 13, 11, 37)
    z.update(mm_a=a, mm_b=b, mm_out=out)
    # fused matmul + bias + gelu
    a, b, bias = rbf((6, 64), 5), rbf((64, 24), 6), rbf((24,), 7)
    out = np.empty((6, 24), np.uint16)
    ref.ref_fused_matmul_bias_gelu(a.ctypes.data, b.ctypes.data, bias.ctypes.data, out.ctypes.data, 6, 24, 64)
    z.update(mbg_a=a, mbg_b=b, mbg_bias=bias, mbg_out=out)
    # gelu over every bf16 code
    allx = np.arange(1 << 16, dtype=np.uint16)
    out = np.empty_like(allx)
    ref.ref_gelu(allx.ctypes.data, out.ctypes.data, allx.size)
    z["gelu_table"] = out
    # softmax
    x = rbf((4, 77), 8, -6, 6)
    out = np.empty_like(x)
    ref.ref_softmax(x.ctypes.data, out.ctypes.data, 4, 77)
    z.update(sm_x=x, sm_out=out)
    with tempfile.TemporaryDirectory() as d:
        d = Path(d)
        # causal attention with a KV prefix
        q, k, v = rbf((1, 2, 5, 32), 9), rbf((1, 2, 12, 32), 10), rbf((1, 2, 12, 32), 11)
        for n, arr in (("q", q), ("k", k), ("v", v)):
            po.save_npy_bf16(d / f"{n}.npy", arr)
        po.run_ref("attention", "prefill", d / "q.npy", d / "k.npy", d / "v.npy", d / "o.npy", "--causal", "1")
        z.update(att_q=q, att_k=k, att_v=v, att_out=po.load_npy_bf16(d / "o.npy").reshape(q.shape))
        # int8 weight-only matmul
        a = rbf((7, 48), 12)
        wq = np.random.default_rng(13).integers(-127, 128, size=(48, 20)).astype(np.int8)
        scale = np.random.default_rng(14).uniform(0.001, 0.02, size=20).astype(np.float32)
        po.save_npy_bf16(d / "a.npy", a)
        np.save(d / "wq.npy", wq)
        np.save(d / "s.npy", scale)
        po.run_ref("matmul_quant", "int8", d / "a.npy", d / "wq.npy", d / "s.npy", d / "c.npy")
        z.update(i8_a=a, i8_wq=wq, i8_scale=scale, i8_out=po.load_npy_bf16(d / "c.npy").reshape(7, 20))
    dst = Path(__file__).resolve().parent / "ref_vectors.npz"
    np.savez_compressed(dst, **z)
    print(f"wrote {dst} ({dst.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
