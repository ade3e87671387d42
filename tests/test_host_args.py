"""Host-side argument handling of the C-ABI, without a GPU.

Every configuration and workspace-size query must answer degenerate shapes
(zero or negative dims) with an error code or 0 -- never abort the process
(the library's error convention: a status and pk_last_error, no abort).
The queries run in a child process so a crash (SIGFPE, SIGSEGV) is reported
as a failure instead of ending the test run.
"""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]

OPS = ["matmul", "fused_matmul_bias_gelu", "fused_matmul_bias_residual", "matmul_int8",
       "matmul_int8_gelu", "matmul_int8_residual", "fused_rmsnorm_matmul", "fused_residual_rmsnorm",
       "fused_softmax_mask", "fused_kv_append_attention"]

_CHILD = r"""
import ctypes as C, itertools, sys
sys.path.insert(0, sys.argv[1])
from polykernel_amd import _lib
lib = C.CDLL(str(_lib.LIB_PATH))
lib.pk_op_configs.argtypes = [C.c_char_p, C.c_longlong, C.c_longlong, C.c_longlong, C.c_void_p, C.c_int]
lib.pk_op_default_config.argtypes = [C.c_char_p, C.c_longlong, C.c_longlong, C.c_longlong, C.POINTER(_lib.Config)]
lib.pk_int8_default_config.argtypes = [C.c_int, C.c_int, C.c_int, C.POINTER(_lib.Config)]
for f in ("pk_mlp_block_workspace_size", "pk_decode_mlp_int8_workspace_size"):
    getattr(lib, f).argtypes = [C.c_int, C.c_int, C.c_int]
    getattr(lib, f).restype = C.c_size_t
dims = [-1, 0, 1, 16, 64, 4096]
ops = sys.argv[2].split(",")
buf = (_lib.Config * 512)()
for op, (m, n, k) in itertools.product(ops, itertools.product(dims, repeat=3)):
    c = _lib.Config()
    rc = lib.pk_op_default_config(op.encode(), m, n, k, C.byref(c))
    cnt = lib.pk_op_configs(op.encode(), m, n, k, buf, 512)
    if min(m, n, k) <= 0 and op.startswith(("matmul", "fused_matmul")):
        assert rc != 0 and cnt == 0, (op, m, n, k, rc, cnt)
for m, n, k in itertools.product(dims, repeat=3):
    c = _lib.Config()
    rc = lib.pk_int8_default_config(m, n, k, C.byref(c))
    if min(m, n, k) <= 0:
        assert rc != 0, (m, n, k)
    for f in ("pk_mlp_block_workspace_size", "pk_decode_mlp_int8_workspace_size"):
        v = getattr(lib, f)(m, n, k)
        if min(m, n, k) <= 0:
            assert v == 0, (f, m, n, k, v)
        else:
            assert v < (1 << 40), (f, m, n, k, v)
print("ok")
"""


def _run_child(ops):
    res = subprocess.run([sys.executable, "-c", _CHILD, str(ROOT), ",".join(ops)],
                         capture_output=True, text=True, timeout=300)
    assert res.returncode == 0 and res.stdout.strip().endswith("ok"), \
        f"child exited {res.returncode}:\n{res.stdout[-2000:]}\n{res.stderr[-2000:]}"


def test_degenerate_shapes_never_abort():
    _run_child(OPS)


def test_int8_zero_k_is_an_error_not_a_crash():
    """pk_op_default_config('matmul_int8', 16, 64, 0) used to divide by a zero
    split length inside the variant planner."""
    import ctypes as C

    from polykernel_amd import _lib

    lib = C.CDLL(str(_lib.LIB_PATH))
    lib.pk_op_default_config.argtypes = [C.c_char_p, C.c_longlong, C.c_longlong, C.c_longlong,
                                         C.POINTER(_lib.Config)]
    lib.pk_last_error.restype = C.c_char_p
    c = _lib.Config()
    assert lib.pk_op_default_config(b"matmul_int8", 16, 64, 0, C.byref(c)) == _lib.PK_ERR_UNSUPPORTED
    assert b"no configuration" in lib.pk_last_error()
    lib.pk_decode_mlp_int8_workspace_size.restype = C.c_size_t
    assert lib.pk_decode_mlp_int8_workspace_size(1, 0, 64) == 0


_GRID_CHILD = r"""
import ctypes as C, sys
sys.path.insert(0, sys.argv[1])
from polykernel_amd import _lib
lib = _lib.load()
P, I, F = C.c_void_p, C.c_int, C.c_float
fake = P(0x100000)  # never dereferenced: every case is refused before a device call
cases = [
    # B * H above INT32_MAX
    ("prefill", (65536, 65536, 1, 1, 128), "exceeds"),
    # (b,h) x query tiles above INT32_MAX workgroups: generic kernel (D 96), wide kernel (D 512), flash (D 128)
    # (128-query tiles: 2^21 x 2^10; 32-query tiles: 2^22 x 2^10; flash 128 x 64 tiles: 2^23 x 2^9)
    ("prefill", (1 << 21, 1, 1 << 17, 1 << 17, 96), "workgroups"),
    ("prefill", (1 << 22, 1, 1 << 15, 1 << 15, 512), "workgroups"),
    ("prefill", (1 << 23, 1, 1 << 16, 64, 128), "workgroups"),
    ("fused", (65536, 65536, 1, 0, 128), "exceeds"),
    # output tilings above INT32_MAX workgroups: GEMM (64 x 64 smallest tile) and RMSNorm -> MatMul (32 x 64)
    ("matmul", (2**31 - 1024, 2**31 - 1024, 64, 0, 0), "workgroups"),
    ("rmsnorm_matmul", (2**31 - 1, 2**30, 64, 0, 0), "INT32_MAX"),
    ("rmsnorm_matmul", (2**31 - 1024, 2**30, 64, 0, 0), "workgroups"),
    # a dimension that rounds up past INT32_MAX
    ("matmul", (2**31 - 1, 8, 32, 0, 0), "INT32_MAX"),
    ("matmul", (1, 8, 2**31 - 8, 0, 0), "INT32_MAX"),
    ("prefill", (1, 1, 2**31 - 1, 16, 64), "INT32_MAX"),
    ("fused", (1, 1, 16, 2**31 - 20, 64), "INT32_MAX"),
]
for kind, (B, H, Sq, Skv, D), word in cases:
    if kind == "prefill":
        rc = lib.launch_attention_prefill(fake, fake, fake, fake, B, H, Sq, Skv, D, F(0.1), 1, None)
    elif kind == "matmul":
        rc = lib.launch_matmul(fake, fake, fake, B, H, Sq, None)
    elif kind == "rmsnorm_matmul":
        rc = lib.launch_fused_rmsnorm_matmul(fake, fake, fake, B, H, Sq, F(1e-6), None)
    else:
        rc = lib.launch_fused_kv_append_attention(fake, fake, fake, fake, fake, fake, B, H, Sq, Skv, D, Sq + Skv,
                                                  F(0.1), 1, None)
    msg = _lib.last_error()
    assert rc < 0 and word in msg, (kind, B, H, Sq, Skv, D, rc, msg)
print("ok")
"""


def test_grid_limits_are_refused_before_launch():
    """Shapes whose grid would overflow the kernels' 32-bit workgroup index
    (attention: B * H, or (b,h) x query tiles x key splits; GEMMs: output
    tiles, above INT32_MAX) return an error before any device call."""
    res = subprocess.run([sys.executable, "-c", _GRID_CHILD, str(ROOT)], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0 and res.stdout.strip().endswith("ok"), \
        f"child exited {res.returncode}:\n{res.stdout[-2000:]}\n{res.stderr[-2000:]}"


_REFUSAL_CHILD = r"""
import ctypes as C, sys
sys.path.insert(0, sys.argv[1])
from polykernel_amd import _lib
from polykernel_amd import runtime as rt
lib = _lib.load()
# launch_matmul_int8_noalloc: split-K partials beyond its 16 MiB static
# buffer are refused before any device call (plausible non-null pointers,
# never dereferenced)
M, N, Kd = 128, 28672, 8192
cfg = rt.default_config("matmul_int8", M, N, Kd)
splits = -(-Kd // cfg["block_k"])
assert splits > 1 and splits * M * N * 4 > (16 << 20), (cfg, splits)
rc = lib.launch_matmul_int8_noalloc(16, 16, 16, 16, M, N, Kd, None)
assert rc == _lib.PK_ERR_WORKSPACE and "static buffer" in _lib.last_error(), (rc, _lib.last_error())
# pk_probe_empty_launch: a geometry outside the device limits is refused
for blocks, threads, lds in ((0, 256, 0), (1, 0, 0), (1, 1025, 0), (1, 64, -1), (1, 64, 160 * 1024 + 4)):
    rc = lib.pk_probe_empty_launch(blocks, threads, lds, None)
    assert rc == _lib.PK_ERR_INVALID_ARG and "pk_probe_empty_launch" in _lib.last_error(), (blocks, threads, lds)
print("ok")
"""


def test_refusals_before_any_device_call():
    """Argument checks that must fail before the library touches a device:
    launch_matmul_int8_noalloc's scratch limit and the launch-floor probe's
    geometry limits (run in a child process, no GPU needed)."""
    res = subprocess.run([sys.executable, "-c", _REFUSAL_CHILD, str(ROOT)], capture_output=True, text=True,
                         timeout=300)
    assert res.returncode == 0 and res.stdout.strip().endswith("ok"), \
        f"child exited {res.returncode}:\n{res.stdout[-2000:]}\n{res.stderr[-2000:]}"
