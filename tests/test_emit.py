"""The gfx950 emitter on the CPU: a tuned int8 entry becomes HIP source that
instantiates the streaming kernel at its config, hipcc --genco cross-compiles
it to an ELF code object, and the KernelCache records and re-checks its
FNV-1a hash (the .hsaco half of lib/Runtime/KernelCache.cpp:296-392)."""
from __future__ import annotations

import json
import shutil

import pytest

from polykernel_amd import _lib
from polykernel_amd import runtime as rt


def int8_entry(op="matmul_int8_gelu", M=16, N=1024, K=2048, config=None):
    cfg = config or rt.default_config(op, M, N, K)
    return {"gpu": "gfx950", "op": op, "shape": {"M": M, "N": N, "K": K, "dtype": "int8"}, "best": cfg,
            "scored_by": "measure", "time_ms": 0.01, "validated": True,
            "correctness": {"cosine": 1.0, "max_rel_err": 0.0, "pcc": 1.0}}


def test_emit_source_instantiates_the_config():
    e = int8_entry(config=dict(block_m=16, block_n=256, block_k=1024, num_warps=4, vector_width=16, unroll=2,
                               shared_memory_stages=6))
    src = rt.emit_source(e)
    assert "pk::i8s::stream_body<4, 1, 4, 6, 1>(g);" in src
    assert "pk::i8s::reduce8_body<1>" in src
    assert "__launch_bounds__(256, 1) void pk_int8_stream(pk_i8s_args g)" in src
    assert "gfx950/matmul_int8_gelu/M=16,N=1024,K=2048,int8" in src


def test_emit_refuses_other_ops_and_foreign_configs():
    gemm = int8_entry()
    gemm.update(op="matmul", shape={"M": 256, "N": 256, "K": 256, "dtype": "bf16"})
    with pytest.raises(rt.RuntimeError_) as ei:
        rt.emit_source(gemm)
    assert "served by the linked kernels" in ei.value.message
    bad = int8_entry()
    bad["best"]["block_n"] = 96
    with pytest.raises(rt.RuntimeError_) as ei:
        rt.emit_source(bad)
    assert "is not one the gfx950 kernels implement" in ei.value.message


@pytest.mark.skipif(shutil.which("hipcc") is None and not __import__("os").path.exists("/opt/rocm/bin/hipcc"),
                    reason="no hipcc")
def test_emit_code_object_records_hash_and_invalidates(tmp_path):
    cache = rt.KernelCache()
    e = int8_entry("matmul_int8_residual", 32, 512, 1024)
    b = rt.emit_code_object(cache, e, tmp_path / "objects")
    so = b["so_path"]
    data = open(so, "rb").read()
    assert data[:4] == b"\x7fELF"
    assert b"pk_int8_stream" in data and b"pk_int8_reduce" in data
    assert b["kernel_hash"] == rt.hash_file(so)
    assert cache.select("gfx950", e["op"], 32, 512, 1024, "int8")["best"] == e["best"]
    # persisted and reloaded
    cache.persist(tmp_path / "cache")
    again = rt.code_object_cache(tmp_path / "cache")
    assert again.get_binary("gfx950", e["op"], 32, 512, 1024, "int8") == b
    # a changed code object is dropped
    with open(so, "ab") as f:
        f.write(b"\0")
    assert again.invalidate_stale() == 1
    assert again.get_binary("gfx950", e["op"], 32, 512, 1024, "int8") is None


def test_code_object_runtime_errors_before_any_device_call(tmp_path):
    """Without a cached code object, and with a mismatched argument block, the
    code-object launcher fails before touching the device."""
    cache = rt.KernelCache()
    e = int8_entry()
    cache.put(e)
    r = rt.Runtime(cache, fixed_arch="gfx950", code_objects=True)
    # non-null placeholders: null operands are refused first (the linked path's check)
    io = rt.MatmulInt8IO(A=16, Wq=16, scale=16, C=16, M=16, N=1024, K=2048)
    with pytest.raises(rt.RuntimeError_) as ei:
        r.run("matmul_int8_gelu", 16, 1024, 2048, io)
    assert "no code object cached" in ei.value.message
    io.K = 4096
    with pytest.raises(rt.RuntimeError_) as ei:
        r.run("matmul_int8_gelu", 16, 1024, 2048, io)
    assert "does not match the selected entry" in ei.value.message


def test_built_code_object_cache_matches_committed_tuning():
    """build() emitted a code object for every int8 entry of the committed cache."""
    if not rt.CODE_OBJECT_DIR.exists():
        pytest.skip("code objects not built (run __graft_entry__.build())")
    cache = rt.code_object_cache()
    doc = json.loads(rt.TUNING_FILE.read_text())
    for e in doc["entries"]:
        sh = e["shape"]
        b = cache.get_binary(e["gpu"], e["op"], sh["M"], sh["N"], sh["K"], sh["dtype"])
        assert (b is not None) == e["op"].startswith("matmul_int8"), e["op"]
        assert cache.select(e["gpu"], e["op"], sh["M"], sh["N"], sh["K"], sh["dtype"])["best"] == e["best"]
