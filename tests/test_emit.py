"""The gfx950 emitter on the CPU: a tuned entry becomes HIP source that
instantiates its op's kernel template at the entry's config, hipcc --genco
cross-compiles it to an ELF code object, and the KernelCache records and
re-checks its FNV-1a hash (the .hsaco half of lib/Runtime/KernelCache.cpp:296-392);
the code-object launchers refuse bad argument blocks before any device call."""
from __future__ import annotations

import json
import shutil

import pytest

from polykernel_amd import _lib, emit
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


def gemm_entry(op="fused_matmul_bias_gelu", M=4096, N=16384, K=4096, config=None):
    cfg = config or rt.default_config(op, M, N, K)
    return {"gpu": "gfx950", "op": op, "shape": {"M": M, "N": N, "K": K, "dtype": "bf16"}, "best": cfg,
            "scored_by": "measure", "time_ms": 0.45, "validated": True,
            "correctness": {"cosine": 1.0, "max_rel_err": 0.0, "pcc": 1.0}}


def test_emit_source_gemm_templates():
    """Each GEMM config names the template it instantiates: the DMA ring
    (block_k 32) at its depth, the register-staged kernels at their tile and
    vector width."""
    src = rt.emit_source(gemm_entry())
    assert "#include \"gemm_kernels.hpp\"" in src
    assert "__launch_bounds__(512, 1) void pk_gemm(pk_gemm_args g)" in src
    assert "pk::gk::gemm_dma_body<1, 5, 8, 4>(g);" in src
    shape = (200, 264, 256)
    for cfg in rt.candidates("fused_matmul_bias_residual", *shape):
        src = rt.emit_source(gemm_entry("fused_matmul_bias_residual", *shape, config=cfg))
        if cfg["block_k"] == 32:
            assert f"gemm_dma_body<2, {cfg['shared_memory_stages']}, 8, 4>" in src
        else:
            wm, wn = (2, 4) if cfg["block_m"] == 256 else (2, 2)
            aligned = "true" if cfg["vector_width"] == 8 else "false"
            assert (f"gemm_reg_body<{cfg['block_m']}, {cfg['block_n']}, {wm}, {wn}, 2, {aligned}>" in src), src
            assert f"__launch_bounds__({64 * cfg['num_warps']}) void pk_gemm" in src


def test_emit_refuses_other_ops_and_foreign_configs():
    other = int8_entry()
    other.update(op="gelu", shape={"M": 64, "N": 4096, "K": 0, "dtype": "bf16"})
    with pytest.raises(rt.RuntimeError_) as ei:
        rt.emit_source(other)
    assert "the emitter instantiates the ops of the tuning cache" in ei.value.message
    bad = int8_entry()
    bad["best"]["block_n"] = 96
    with pytest.raises(rt.RuntimeError_) as ei:
        rt.emit_source(bad)
    assert "is not one the gfx950 kernels implement" in ei.value.message


def row_entry(op, rows, cols):
    dtype = "fp32" if op == "fused_softmax_mask" else "bf16"
    return {"gpu": "gfx950", "op": op, "shape": {"M": rows, "N": cols, "K": 0, "dtype": dtype},
            "best": rt.default_config(op, rows, cols, 0), "scored_by": "model", "time_ms": None, "validated": True,
            "correctness": {"cosine": 1.0, "max_rel_err": 0.0, "pcc": 1.0}}


def test_emit_source_row_templates():
    """Each row config instantiates the kernel rowwise.hip's dispatcher runs
    for that width (waves per row, vectors per lane), with the generic kernel
    as the second entry point for unaligned operands."""
    for op, body, any_ in (("fused_residual_rmsnorm", "rmsnorm_vec_body", "rmsnorm_generic_body<true>"),
                           ("fused_softmax_mask", "softmax_vec_body", "softmax_generic_body<1>")):
        rms = op == "fused_residual_rmsnorm"
        kind = "true" if rms else "1"
        # built-in choices: one wave per row for short rows, then a row per
        # workgroup of 4 or 8 waves (8 for softmax, and for RMSNorm above 1024 vectors)
        widths = {512: (1, 1), 1024: (1, 2), 4096: (1, 8) if rms else (8, 1), 8192: (4, 4) if rms else (8, 2),
                  16384: (8, 4), 32768: (16, 4), 65536: (16, 8)}
        for cols, (nw, vpt) in widths.items():
            src = rt.emit_source(row_entry(op, 64, cols))
            threads = 256 if nw <= 4 else 64 * nw
            assert (f"__launch_bounds__({threads}) void pk_row(pk_row_args a) {{\n  "
                    f"pk::row::{body}<{nw}, {vpt}, {kind}>(a);") in src, (op, cols, src)
            assert f"void pk_row_any(pk_row_args a) {{\n  pk::row::{any_}(a);" in src, (op, cols)
            assert '#include "rowwise_kernels.hpp"' in src
        for cols in (70000, 131072):  # 65537-131072 columns: the packed-bf16 kernel
            src = rt.emit_source(row_entry(op, 64, cols))
            assert f"__launch_bounds__(1024) void pk_row(pk_row_args a) {{\n  pk::row::{body.replace('vec', 'packed')}<{kind}>(a);" in src, cols
        for cols in (999, 140000):  # cols % 8 != 0, and rows longer than 131072 columns
            src = rt.emit_source(row_entry(op, 64, cols))
            assert f"void pk_row(pk_row_args a) {{\n  pk::row::{any_}(a);" in src, cols
        # every candidate of a long row (4, 8 and 16 waves) has a template
        for cols in (4096, 8192, 16384, 32768, 40000, 65536):
            e = row_entry(op, 64, cols)
            for cfg in rt.candidates(op, 64, cols, 0):
                e["best"] = cfg
                assert f"vec_body<{cfg['num_warps'] if cfg['block_m'] == 1 else 1}, {cfg['unroll']}, {kind}>" in \
                    rt.emit_source(e), (op, cols, cfg)


def test_emit_source_rmsnorm_matmul_templates():
    """fused_rmsnorm_matmul: the whole-K panel (K <= 832, one round of tiles)
    and, otherwise, RMSNorm at the (M, K) row config followed by the config's
    GEMM."""
    src = rt.emit_source(gemm_entry("fused_rmsnorm_matmul", 128, 3072, 768))
    assert "__launch_bounds__(512) void pk_panel(pk_panel_args a) {\n  pk::gk::rmsnorm_panel_fast_body(a);" in src
    # past one round of panel tiles (M 300, N 4096): RMSNorm into workspace and the GEMM
    assert "pk_panel" not in rt.emit_source(gemm_entry("fused_rmsnorm_matmul", 300, 4096, 768))
    e = gemm_entry("fused_rmsnorm_matmul", 72, 264, 2048)
    src = rt.emit_source(e)
    assert "pk::row::rmsnorm_vec_body<1, 4, false>(a);" in src and "rmsnorm_generic_body<false>(a);" in src
    c = e["best"]
    assert f"gemm_reg_body<{c['block_m']}, {c['block_n']}, 2, 2, 0, true>(g);" in src, src
    assert "void pk_gemm(pk_gemm_args g)" in src


def test_emit_source_rmsnorm_matmul_k64_gemm_configs_are_not_panels():
    """At K = 64 the 64-deep GEMM configs (block_k 64, 4 waves) have
    block_k == K like the panel config; only the 32 x 64 tile (8 waves) is the panel.
    Every GEMM candidate must emit pk_gemm (the panel kernel needs N % 8 == 0
    and one round of tiles), and the panel candidate pk_panel."""
    for shape in ((4096, 1001, 64), (4096, 512, 64), (64, 256, 64)):
        for cfg in rt.candidates("fused_rmsnorm_matmul", *shape):
            src = rt.emit_source(gemm_entry("fused_rmsnorm_matmul", *shape, config=cfg))
            panel = (cfg["block_m"], cfg["block_n"], cfg["block_k"]) == (32, 64, shape[2])
            assert ("void pk_panel(" in src) == panel, (shape, cfg)
            assert ("void pk_gemm(" in src) == (not panel), (shape, cfg)
    # the small shape fits the panel, so its candidates include it
    assert any((c["block_m"], c["block_n"]) == (32, 64) for c in rt.candidates("fused_rmsnorm_matmul", 64, 256, 64))


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
    """build() emitted a code object for every entry of the committed cache."""
    if not rt.CODE_OBJECT_DIR.exists():
        pytest.skip("code objects not built (run __graft_entry__.build())")
    cache = rt.code_object_cache()
    doc = json.loads(rt.TUNING_FILE.read_text())
    for e in doc["entries"]:
        sh = e["shape"]
        b = cache.get_binary(e["gpu"], e["op"], sh["M"], sh["N"], sh["K"], sh["dtype"])
        assert (b is not None) == (e["op"] in emit.EMIT_OPS), e["op"]
        assert cache.select(e["gpu"], e["op"], sh["M"], sh["N"], sh["K"], sh["dtype"])["best"] == e["best"]


def test_conformance_objects_built():
    """build() emitted every GEMM template (each epilogue) and int8 variant of
    the conformance set; each manifest line names an ELF whose hash matches."""
    m = emit.CONFORMANCE_OUT / "manifest.json"
    if not m.exists():
        pytest.skip("conformance objects not built (run __graft_entry__.build())")
    lines = json.loads(m.read_text())
    assert len(lines) == len(emit.conformance_entries())
    assert len({l["so_path"] for l in lines}) == len(lines)  # one object per (op, config)
    for l in lines:
        data = open(l["so_path"], "rb").read(4)
        assert data == b"\x7fELF"
        assert rt.hash_file(l["so_path"]) == l["kernel_hash"]


def test_code_object_gemm_launcher_checks_before_any_device_call():
    """Null operands, a shape other than the entry's and misaligned operands
    for a 16-byte config are refused without touching the device."""
    cache = rt.KernelCache()
    e = gemm_entry()
    cache.put(e)
    r = rt.Runtime(cache, fixed_arch="gfx950", code_objects=True)
    io = rt.MatmulIO(A=256, B=256, C=256, bias=None, residual=None, M=4096, N=16384, K=4096)
    with pytest.raises(rt.RuntimeError_) as ei:
        r.run("fused_matmul_bias_gelu", 4096, 16384, 4096, io)
    assert "null tensor pointer" in ei.value.message
    io.bias = 256
    io.A = 258  # not 16-byte aligned
    with pytest.raises(rt.RuntimeError_) as ei:
        r.run("fused_matmul_bias_gelu", 4096, 16384, 4096, io)
    assert "16-byte aligned" in ei.value.message
    io.A = 256
    with pytest.raises(rt.RuntimeError_) as ei:
        r.run("fused_matmul_bias_gelu", 4096, 16384, 4096, io)
    assert "no code object cached" in ei.value.message


def test_code_object_row_and_panel_launchers_check_before_any_device_call():
    """Null operands, a shape other than the entry's, and (panel configs)
    misaligned operands are refused without touching the device; row objects
    take unaligned operands on their generic entry point, so for them the
    next refusal is the missing code object."""
    cache = rt.KernelCache()
    cache.put(row_entry("fused_residual_rmsnorm", 64, 4096))
    cache.put(row_entry("fused_softmax_mask", 64, 4096))
    cache.put(gemm_entry("fused_rmsnorm_matmul", 128, 3072, 768))
    r = rt.Runtime(cache, fixed_arch="gfx950", code_objects=True)
    io = rt.ResidualRmsnormIO(x=256, r=None, gamma=None, out=256, rows=64, cols=4096, eps=1e-6)
    with pytest.raises(rt.RuntimeError_) as ei:
        r.run("fused_residual_rmsnorm", 64, 4096, 0, io)
    assert "null tensor pointer" in ei.value.message
    io.r = 258
    with pytest.raises(rt.RuntimeError_) as ei:
        r.run("fused_residual_rmsnorm", 64, 4096, 0, io)
    assert "no code object cached" in ei.value.message
    io.cols = 2048
    with pytest.raises(rt.RuntimeError_) as ei:
        r.run("fused_residual_rmsnorm", 64, 4096, 0, io)
    assert "does not match the selected entry" in ei.value.message
    sio = rt.SoftmaxMaskIO(logits=256, mask=None, out=256, rows=64, cols=4096)
    with pytest.raises(rt.RuntimeError_) as ei:
        r.run("fused_softmax_mask", 64, 4096, 0, sio)
    assert "null tensor pointer" in ei.value.message
    pio = rt.RmsnormMatmulIO(x=256, gamma=None, W=None, out=256, M=128, N=3072, K=768, eps=1e-6)
    with pytest.raises(rt.RuntimeError_) as ei:
        r.run("fused_rmsnorm_matmul", 128, 3072, 768, pio)
    assert "null tensor pointer" in ei.value.message
    pio.W = 264  # not 16-byte aligned
    with pytest.raises(rt.RuntimeError_) as ei:
        r.run("fused_rmsnorm_matmul", 128, 3072, 768, pio)
    assert "16-byte aligned" in ei.value.message
    pio.W = 256
    with pytest.raises(rt.RuntimeError_) as ei:
        r.run("fused_rmsnorm_matmul", 128, 3072, 768, pio)
    assert "no code object cached" in ei.value.message


def att_entry(S_q=512, S_kv=4096, D=128, config=None):
    cfg = config or rt.default_config("fused_kv_append_attention", S_q, S_kv, D)
    return {"gpu": "gfx950", "op": "fused_kv_append_attention", "shape": {"M": S_q, "N": S_kv, "K": D, "dtype": "bf16"},
            "best": cfg, "scored_by": "measure", "time_ms": 0.06, "validated": True,
            "correctness": {"cosine": 1.0, "max_rel_err": 0.0, "pcc": 1.0}}


def test_emit_source_attention_templates():
    """Flash tile shapes instantiate the fused flash kernel and its merge; the
    generic config the generic kernel (both alignments), its merge and the
    in-place append."""
    for cfg in rt.candidates("fused_kv_append_attention", 512, 4096, 128):
        src = rt.emit_source(att_entry(config=cfg))
        qg = cfg["block_m"] // 32
        assert f"pk::att::fa_body<128, {qg}, true>(g);" in src
        assert "void pk_fa_combine(pk_fa_args g)" in src and "pk::att::fa_combine_body<128>" in src
    (gen,) = rt.candidates("fused_kv_append_attention", 100, 300, 200)
    src = rt.emit_source(att_entry(100, 300, 200, gen))
    for want in ("pk::att::att_body<256, true>(g);", "pk::att::att_body<256, false>(g);",
                 "pk::att::att_combine_body<256>(g);", "pk::att::kv_append_body(a);"):
        assert want in src


def test_code_object_attention_launcher_checks_before_any_device_call():
    cache = rt.KernelCache()
    cache.put(att_entry())
    r = rt.Runtime(cache, fixed_arch="gfx950", code_objects=True)
    io = rt.KvAppendAttentionIO(Q=256, Kc=256, Vc=256, Kn=None, Vn=256, O=256, B=1, H=32, S_q=512, S_cache=3584,
                                D=128, cache_capacity=4096, scale=0.088, causal=1)
    with pytest.raises(rt.RuntimeError_) as ei:
        r.run("fused_kv_append_attention", 512, 4096, 128, io)
    assert "null tensor pointer" in ei.value.message
    io.Kn = 256
    with pytest.raises(rt.RuntimeError_) as ei:
        r.run("fused_kv_append_attention", 512, 4096, 128, io)
    assert "no code object cached" in ei.value.message
