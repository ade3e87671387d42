"""Runtime layer on the CPU: the tuning-cache document, KernelCache
(select / persist / binary hashing / stale invalidation), the correctness
gate, the gfx950 config space and Runtime's detect -> select path.

Mirrors the reference's own unit tests of these classes
(lib/Autotune/tests/{tuning_cache,amd_tuning_db,benchmark}_test.cpp,
lib/Runtime/tests/{runtime,kernel_cache_persist,device_detect}_test.cpp):
same cases, same expected error fragments.  Nothing here launches a kernel.
"""
from __future__ import annotations

import copy
import json
import math
import os

import pytest

from polykernel_amd import _lib
from polykernel_amd import runtime as rt

SHAPE = dict(M=2048, N=4096, K=11008, dtype="bf16")
OP = "fused_matmul_bias_gelu"


def entry(gpu="gfx950", op=OP, shape=SHAPE, validated=True, time_ms=0.123, block_m=256):
    return {
        "gpu": gpu, "op": op, "shape": dict(shape),
        "best": {"block_m": block_m, "block_n": 256, "block_k": 32, "num_warps": 4,
                 "vector_width": 8, "unroll": 2, "shared_memory_stages": 5},
        "scored_by": "measure", "time_ms": time_ms, "validated": validated,
        "correctness": {"cosine": 0.9999, "max_rel_err": 1e-4, "pcc": 0.999},
    }


def doc(*entries):
    return json.dumps({"version": 1, "entries": list(entries)})


def key_args(gpu="gfx950", op=OP, shape=SHAPE):
    return (gpu, op, shape["M"], shape["N"], shape["K"], shape["dtype"])


# ---- tuning-cache document ---------------------------------------------------------

def test_roundtrip_measured_and_modeled():
    c = rt.KernelCache()
    modeled = entry(gpu="gfx942", shape=dict(M=128, N=128, K=128, dtype="fp16"), validated=False, time_ms=None)
    modeled["scored_by"] = "compile_time_model"
    c.load_tuning_cache(doc(entry(), modeled))
    text = c.serialize()
    assert '"time_ms":null' in text and '"time_ms":0.123' in text
    back = json.loads(text)
    assert back["version"] == 1
    got = sorted(back["entries"], key=lambda e: e["gpu"])
    assert got == sorted([entry(), modeled], key=lambda e: e["gpu"])
    # serialising the reparsed document gives the same bytes (canonical form)
    c2 = rt.KernelCache()
    c2.load_tuning_cache(text)
    assert c2.serialize() == text


def test_serialised_form_is_compact_with_sorted_keys():
    c = rt.KernelCache()
    c.load_tuning_cache(doc(entry()))
    text = c.serialize()
    assert text.startswith('{"entries":[{"best":{"block_k":32,"block_m":256,')
    assert text.endswith('"version":1}')
    assert " " not in text


@pytest.mark.parametrize("mutate,fragment", [
    (lambda e: e.pop("scored_by"), "entries[0].scored_by: missing required string field"),
    (lambda e: e["correctness"].pop("cosine"), "entries[0].correctness.cosine: missing required number field"),
    (lambda e: e.pop("time_ms"), "entries[0].time_ms: missing required field"),
    (lambda e: e.__setitem__("validated", "yes"), "entries[0].validated: expected a boolean"),
    (lambda e: e["best"].__setitem__("block_k", 3.5), "entries[0].best.block_k: expected an integer"),
    (lambda e: e["shape"].pop("dtype"), "entries[0].shape.dtype: missing required string field"),
    (lambda e: e.__setitem__("time_ms", "fast"), "entries[0].time_ms: expected a number or null"),
    (lambda e: e.__setitem__("gpu", ""), "entries[0].gpu: empty gpu"),
])
def test_schema_errors_name_the_field(mutate, fragment):
    e = entry()
    mutate(e)
    c = rt.KernelCache()
    with pytest.raises(rt.RuntimeError_) as ei:
        c.load_tuning_cache(doc(e))
    assert fragment in ei.value.message


@pytest.mark.parametrize("text,fragment", [
    ('{"version": 2, "entries": []}', "root.version: unsupported schema version 2 (expected 1)"),
    ('{"entries": []}', "root.version: missing required integer field"),
    ('{"version": 1}', "root.entries: missing required array field"),
    ('{"version": 1, "entries": {}}', "root.entries: expected an array"),
    ('[1, 2]', "root: expected a JSON object"),
    ('{"version": 1, "entries": [1]}', "entries[0]: expected an object"),
    ('{"version": 1, "entries": [}', "malformed JSON"),
    ('{"version": 1, "entries": [],}', "malformed JSON"),
    ('{"version": 1, "version": 1, "entries": []}', "malformed JSON"),
    ('{"version": 1, "entries": []} x', "malformed JSON"),
])
def test_envelope_errors(text, fragment):
    c = rt.KernelCache()
    with pytest.raises(rt.RuntimeError_) as ei:
        c.load_tuning_cache(text)
    assert fragment in ei.value.message


def test_integral_float_reads_as_integer_and_unknown_members_are_ignored():
    e = entry()
    e["shape"]["M"] = 2048.0
    e["note"] = "extra members are ignored, as the reference parser ignores them"
    c = rt.KernelCache()
    c.load_tuning_cache(doc(e))
    assert c.select(*key_args())["shape"]["M"] == 2048


def test_failed_load_leaves_previous_entries():
    c = rt.KernelCache()
    c.load_tuning_cache(doc(entry()))
    with pytest.raises(rt.RuntimeError_):
        c.load_tuning_cache('{"version": 1, "entries": [{}]}')
    assert len(c) == 1


# ---- selection ---------------------------------------------------------------------------

def test_select_validated_entry():
    c = rt.KernelCache()
    c.load_tuning_cache(doc(entry()))
    got = c.select(*key_args())
    assert got == entry()


def test_miss_is_clear_error():
    c = rt.KernelCache()
    c.load_tuning_cache(doc(entry()))
    with pytest.raises(rt.RuntimeError_) as ei:
        c.select("gfx950", OP, 128, 128, 128, "bf16")
    msg = ei.value.message
    assert ei.value.code == _lib.PK_ERR_NOT_FOUND
    assert "no tuned kernel for gfx950/fused_matmul_bias_gelu/M=128,N=128,K=128,bf16" in msg
    assert "run the autotuner" in msg


def test_unvalidated_entry_is_not_served():
    c = rt.KernelCache()
    c.load_tuning_cache(doc(entry(validated=False)))
    with pytest.raises(rt.RuntimeError_) as ei:
        c.select(*key_args())
    assert "not validated" in ei.value.message and "run the autotuner" in ei.value.message


def test_namespaces_are_isolated_and_last_writer_wins():
    c = rt.KernelCache()
    c.put(entry(gpu="gfx942", block_m=64))
    with pytest.raises(rt.RuntimeError_):
        c.select(*key_args(gpu="gfx950"))
    c.put(entry(gpu="gfx950", block_m=128))
    c.put(entry(gpu="gfx950", block_m=256))
    assert len(c) == 2
    assert c.select(*key_args(gpu="gfx950"))["best"]["block_m"] == 256
    assert c.select(*key_args(gpu="gfx942"))["best"]["block_m"] == 64


def test_format_key():
    assert rt.format_key("gfx950", "matmul", 4096, 4096, 4096, "bf16") == "gfx950/matmul/M=4096,N=4096,K=4096,bf16"


# ---- binaries: FNV-1a, persistence, invalidation -----------------------------------------------

# The reference seeds its FNV-1a 64 with 1469598103934665603
# (lib/Runtime/KernelCache.cpp:56) -- one decimal digit short of the published
# offset basis 14695981039346656037.  Hashes have to agree with the
# binaries.json files the reference writes, so the library keeps its constant.
REFERENCE_BASIS = 1469598103934665603
FNV_BASIS = 14695981039346656037
FNV_PRIME = 1099511628211


def _fnv1a64(data: bytes, basis: int = REFERENCE_BASIS) -> str:
    h = basis
    for b in data:
        h = ((h ^ b) * FNV_PRIME) & 0xFFFFFFFFFFFFFFFF
    return f"{h:016x}"


@pytest.mark.parametrize("data,expected", [
    (b"", "cbf29ce484222325"),       # published FNV-1a 64 test vectors: they pin
    (b"a", "af63dc4c8601ec8c"),      # the xor-then-multiply order and the prime
    (b"foobar", "85944171f73967e8"),
])
def test_fnv1a_restatement_known_vectors(data, expected):
    assert _fnv1a64(data, FNV_BASIS) == expected


@pytest.mark.parametrize("data", [b"", b"a", b"foobar", bytes(range(256)) * 3])
def test_hash_file_matches_reference_fnv(tmp_path, data):
    p = tmp_path / "f.bin"
    p.write_bytes(data)
    assert rt.hash_file(p) == _fnv1a64(data)
    if not data:
        assert rt.hash_file(p) == f"{REFERENCE_BASIS:016x}" == "14650fb0739d0383"


def test_hash_file_large_and_missing(tmp_path):
    p = tmp_path / "big.bin"
    data = os.urandom(200_000)
    p.write_bytes(data)
    assert rt.hash_file(p) == _fnv1a64(data)
    with pytest.raises(rt.RuntimeError_) as ei:
        rt.hash_file(tmp_path / "nope.so")
    assert "cannot read binary" in ei.value.message


def _with_binary(tmp_path, content=b"code-object-v1"):
    so = tmp_path / "gfx950.hsaco"
    so.write_bytes(content)
    c = rt.KernelCache()
    c.put(entry())
    c.put_binary(*key_args(), str(so), rt.hash_file(so))
    return c, so


def test_binary_must_back_an_entry(tmp_path):
    c = rt.KernelCache()
    with pytest.raises(rt.RuntimeError_):
        c.put_binary(*key_args(), str(tmp_path / "x.hsaco"), "0" * 16)


def test_persist_then_reload(tmp_path):
    c, so = _with_binary(tmp_path)
    c.persist(tmp_path / "cache")
    assert sorted(os.listdir(tmp_path / "cache")) == ["binaries.json", "tuning_db.json"]
    r = rt.KernelCache()
    r.load_persisted(tmp_path / "cache")
    assert len(r) == 1
    assert r.select(*key_args())["best"]["block_m"] == 256
    b = r.get_binary(*key_args())
    assert b["so_path"] == str(so) and b["kernel_hash"] == rt.hash_file(so)


def test_stale_binary_invalidated(tmp_path):
    c, so = _with_binary(tmp_path)
    assert c.invalidate_stale() == 0
    so.write_bytes(b"code-object-v2")
    assert c.invalidate_stale() == 1
    assert c.get_binary(*key_args()) is None
    with pytest.raises(rt.RuntimeError_) as ei:
        c.select(*key_args())
    assert "no tuned kernel" in ei.value.message


def test_missing_binary_invalidated(tmp_path):
    c, so = _with_binary(tmp_path)
    so.unlink()
    assert c.invalidate_stale() == 1
    assert len(c) == 0


def test_entries_without_binaries_survive_invalidation(tmp_path):
    c, so = _with_binary(tmp_path)
    c.put(entry(op="matmul"))
    so.unlink()
    assert c.invalidate_stale() == 1
    assert c.select(*key_args(op="matmul"))["op"] == "matmul"


def test_load_persisted_rejects_malformed_binaries(tmp_path):
    c, so = _with_binary(tmp_path)
    d = tmp_path / "cache"
    c.persist(d)
    bins = json.loads((d / "binaries.json").read_text())
    del bins["binaries"][0]["so_path"]
    (d / "binaries.json").write_text(json.dumps(bins))
    r = rt.KernelCache()
    r.put(entry(op="matmul"))
    with pytest.raises(rt.RuntimeError_) as ei:
        r.load_persisted(d)
    assert "binaries.json: binaries[0].so_path: missing required string field" in ei.value.message
    assert len(r) == 1  # unchanged on failure


def test_load_persisted_rejects_orphan_binary(tmp_path):
    c, so = _with_binary(tmp_path)
    d = tmp_path / "cache"
    c.persist(d)
    (d / "tuning_db.json").write_text(doc())
    with pytest.raises(rt.RuntimeError_) as ei:
        rt.KernelCache().load_persisted(d)
    assert "a binary must back a present tuning entry" in ei.value.message


# ---- gate and selection ---------------------------------------------------------------------------

def test_gate_thresholds():
    g = rt.passes_correctness_gate
    assert g(0.999, 1e-2, 0.99)
    assert not g(0.9989, 0.0, 1.0)
    assert not g(1.0, 0.0, 0.9899)
    assert not g(1.0, 0.011, 1.0)
    assert g(1.0, 0.04, 1.0, 5e-2)
    assert not g(float("nan"), 0.0, 1.0)
    assert not g(1.0, float("nan"), 1.0, math.inf)
    assert g(1.0, 1e300, 1.0, math.inf)


def test_rel_ceiling_follows_reference_rule():
    assert rt.rel_ceiling("matmul", 255) == 1e-2
    assert math.isinf(rt.rel_ceiling("matmul", 256))
    assert math.isinf(rt.rel_ceiling("fused_matmul_bias_gelu", 64))


def test_select_best_validated():
    s = rt.select_best_validated
    assert s([]) is None
    assert s([(False, None), (False, None)]) is None
    assert s([(True, 3.0), (True, 1.0), (True, 2.0)]) == 1
    assert s([(True, 2.0), (False, 0.5), (True, 2.5)]) == 0  # never the faster unvalidated one
    assert s([(True, 1.0), (True, 1.0)]) == 0                  # ties: lowest index
    assert s([(True, None), (True, 4.0)]) == 1                 # validated but untimed is no candidate


# ---- config space -----------------------------------------------------------------------------------

BASELINE_SHAPES = [
    ("fused_rmsnorm_matmul", 128, 3072, 768),
    ("fused_matmul_bias_gelu", 4096, 16384, 4096),
    ("fused_matmul_bias_residual", 4096, 4096, 16384),
    ("fused_kv_append_attention", 512, 4096, 128),
    ("fused_residual_rmsnorm", 16384, 8192, 0),
    ("fused_softmax_mask", 16384, 8192, 0),
    ("matmul_int8_gelu", 16, 28672, 8192),
    ("matmul_int8_residual", 16, 8192, 28672),
]


@pytest.mark.parametrize("op,M,N,K", BASELINE_SHAPES)
def test_every_baseline_shape_has_candidates_and_default_among_them(op, M, N, K):
    cands = rt.candidates(op, M, N, K)
    assert cands, op
    assert len({json.dumps(c, sort_keys=True) for c in cands}) == len(cands)
    d = rt.default_config(op, M, N, K)
    assert d in cands
    for c in cands:
        assert c["num_warps"] * 64 <= 1024
        assert all(c[f] > 0 for f in ("block_m", "block_n", "num_warps", "vector_width", "unroll",
                                      "shared_memory_stages"))


def test_int8_candidates_cover_variants_and_splits():
    cands = rt.candidates("matmul_int8", 16, 28672, 8192)
    assert {c["vector_width"] for c in cands} == {16} and {c["unroll"] for c in cands} == {2}
    assert {c["block_m"] for c in cands} == {16}
    splits = {8192 // c["block_k"] for c in cands if 8192 % c["block_k"] == 0}
    assert {1, 2, 4, 8, 16, 32} <= splits
    for c in cands:  # LDS of the per-wave rings fits the CU
        nt = c["block_n"] // (16 * c["num_warps"])
        assert c["shared_memory_stages"] * c["num_warps"] * 1024 * (nt + 2) <= 160 * 1024
    # more row blocks are offered once M grows
    assert {c["block_m"] for c in rt.candidates("matmul_int8", 64, 4096, 4096)} == {16, 32, 64}


def test_gemm_candidates_depend_on_shape():
    big = rt.candidates("matmul", 4096, 4096, 4096)
    assert [c["shared_memory_stages"] for c in big[:2]] == [5, 4] and big[0]["block_k"] == 32
    odd = rt.candidates("matmul", 130, 127, 65)  # no DMA ring, element-wise loads only
    assert odd and all(c["vector_width"] == 1 and c["shared_memory_stages"] == 2 for c in odd)


def test_config_space_rejects_unknown_op_and_wrong_dtype():
    with pytest.raises(rt.RuntimeError_):
        rt.default_config("conv2d", 1, 1, 1)
    assert rt.candidates("matmul", 64, 64, 64, dtype="fp16") == []
    assert rt.candidates("fused_residual_rmsnorm", 64, 64, 7) == []


# ---- runtime: detect -> select ----------------------------------------------------------------------

def test_runtime_resolves_for_detected_arch():
    c = rt.KernelCache()
    c.put(entry(gpu="gfx942", block_m=64))
    c.put(entry(gpu="gfx950", block_m=256))
    r = rt.Runtime(c, fixed_arch="gfx950")
    assert r.resolve(OP, SHAPE["M"], SHAPE["N"], SHAPE["K"])["best"]["block_m"] == 256
    r942 = rt.Runtime(c, fixed_arch="gfx942")
    assert r942.resolve(OP, SHAPE["M"], SHAPE["N"], SHAPE["K"])["best"]["block_m"] == 64


def test_runtime_miss_on_other_arch_and_untuned_shape():
    c = rt.KernelCache()
    c.put(entry())
    with pytest.raises(rt.RuntimeError_) as ei:
        rt.Runtime(c, fixed_arch="gfx900").resolve(OP, SHAPE["M"], SHAPE["N"], SHAPE["K"])
    assert "no tuned kernel" in ei.value.message and "gfx900" in ei.value.message
    with pytest.raises(rt.RuntimeError_) as ei:
        rt.Runtime(c, fixed_arch="gfx950").resolve(OP, 128, 128, 128)
    assert "M=128,N=128,K=128" in ei.value.message


def test_runtime_refuses_mismatched_argument_block():
    """The launcher checks the io block against the selected shape before
    any device call (so this runs without a GPU)."""
    c = rt.KernelCache()
    e = entry(op="fused_matmul_bias_gelu", shape=dict(M=4096, N=16384, K=4096, dtype="bf16"))
    c.put(e)
    r = rt.Runtime(c, fixed_arch="gfx950")
    io = rt.MatmulIO(M=4096, N=16384, K=1024)
    with pytest.raises(rt.RuntimeError_) as ei:
        r.run("fused_matmul_bias_gelu", 4096, 16384, 4096, io)
    assert "does not match the selected entry" in ei.value.message


def test_runtime_refuses_config_the_kernels_lack():
    c = rt.KernelCache()
    e = entry(op="fused_matmul_bias_gelu", shape=dict(M=4096, N=16384, K=4096, dtype="bf16"))
    e["best"]["block_m"] = 96
    c.put(e)
    r = rt.Runtime(c, fixed_arch="gfx950")
    io = rt.MatmulIO(M=4096, N=16384, K=4096)
    with pytest.raises(rt.RuntimeError_) as ei:
        r.run("fused_matmul_bias_gelu", 4096, 16384, 4096, io)
    assert "is not one the gfx950 kernels implement" in ei.value.message


def test_hip_detector_without_gpu_reports_detection_failure():
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    c = rt.KernelCache()
    c.put(entry())
    with pytest.raises(rt.RuntimeError_) as ei:
        rt.Runtime(c).resolve(OP, SHAPE["M"], SHAPE["N"], SHAPE["K"])
    assert ei.value.code == _lib.PK_ERR_NO_DEVICE
    assert "device detection failed" in ei.value.message


def test_code_object_int8_launcher_rejects_null_operands():
    """The code-object int8 launcher refuses null operands before loading or
    launching anything, with the linked path's wording (no GPU needed)."""
    c = rt.KernelCache()
    shape = dict(M=16, N=28672, K=8192, dtype="int8")
    e = entry(op="matmul_int8_gelu", shape=shape)
    e["best"] = {"block_m": 16, "block_n": 512, "block_k": 2048, "num_warps": 4,
                 "vector_width": 16, "unroll": 2, "shared_memory_stages": 3}
    c.put(e)
    r = rt.Runtime(c, fixed_arch="gfx950", code_objects=True)
    for missing in ("A", "Wq", "scale", "C"):
        io = rt.MatmulInt8IO(A=16, Wq=16, scale=16, C=16, M=16, N=28672, K=8192)
        setattr(io, missing, None)
        with pytest.raises(rt.RuntimeError_) as ei:
            r.run("matmul_int8_gelu", 16, 28672, 8192, io)
        assert "null tensor pointer" in ei.value.message, ei.value.message


# ---- code-object launchers: refusals before any device call -----------------------
# Each launcher served from an emitted code object checks its argument block the
# way the linked path does (null operands, the entry's shape, the operand alignment
# its config needs, a cached binary) before it loads a module or launches, so these
# run without a GPU.  Pointers are fake, nonzero addresses: nothing dereferences them.

GEMM_DMA = {"block_m": 256, "block_n": 256, "block_k": 32, "num_warps": 8,
            "vector_width": 8, "unroll": 2, "shared_memory_stages": 5}
PANEL = {"block_m": 32, "block_n": 64, "block_k": 768, "num_warps": 8,
         "vector_width": 8, "unroll": 48, "shared_memory_stages": 1}
ROW = {"block_m": 1, "block_n": 8192, "block_k": 0, "num_warps": 4,
       "vector_width": 8, "unroll": 4, "shared_memory_stages": 1}
FLASH = {"block_m": 64, "block_n": 128, "block_k": 128, "num_warps": 8,
         "vector_width": 8, "unroll": 8, "shared_memory_stages": 2}


def _object_runtime(op, shape, best):
    c = rt.KernelCache()
    e = entry(op=op, shape=dict(shape, dtype=rt.op_dtype(op)))
    e["best"] = dict(best)
    c.put(e)
    return rt.Runtime(c, fixed_arch="gfx950", code_objects=True)


def _refused(r, op, mnk, io, fragment):
    with pytest.raises(rt.RuntimeError_) as ei:
        r.run(op, *mnk, io)
    assert fragment in ei.value.message, ei.value.message


@pytest.mark.parametrize("op,needs", [("matmul", ("A", "B", "C")),
                                      ("fused_matmul_bias_gelu", ("A", "B", "C", "bias")),
                                      ("fused_matmul_bias_residual", ("A", "B", "C", "residual"))])
def test_code_object_gemm_launcher_refusals(op, needs):
    mnk = (512, 512, 256)
    r = _object_runtime(op, dict(M=512, N=512, K=256), GEMM_DMA)
    ok = dict(A=4096, B=8192, C=12288, bias=16384, residual=20480, M=512, N=512, K=256)
    for missing in needs:
        io = rt.MatmulIO(**ok)
        setattr(io, missing, None)
        _refused(r, op, mnk, io, "code object: null tensor pointer")
    _refused(r, op, mnk, rt.MatmulIO(**dict(ok, K=128)), "does not match the selected entry")
    _refused(r, op, mnk, rt.MatmulIO(**dict(ok, A=4098)), "needs 16-byte aligned A and B")
    _refused(r, op, mnk, rt.MatmulIO(**dict(ok, C=12290)), "needs 16-byte aligned C, residual and bias")
    # every check passed: the cache holds no binary for the entry
    _refused(r, op, mnk, rt.MatmulIO(**ok), "no code object cached")


def test_code_object_panel_launcher_refusals():
    op, mnk = "fused_rmsnorm_matmul", (128, 3072, 768)
    r = _object_runtime(op, dict(M=128, N=3072, K=768), PANEL)
    ok = dict(x=4096, gamma=8192, W=12288, out=16384, M=128, N=3072, K=768, eps=1e-6)
    for missing in ("x", "W", "out"):
        io = rt.RmsnormMatmulIO(**ok)
        setattr(io, missing, None)
        _refused(r, op, mnk, io, "code object: null tensor pointer")
    _refused(r, op, mnk, rt.RmsnormMatmulIO(**dict(ok, N=2048)), "does not match the selected entry")
    _refused(r, op, mnk, rt.RmsnormMatmulIO(**dict(ok, gamma=8194)), "needs 16-byte aligned x, W, gamma and out")
    _refused(r, op, mnk, rt.RmsnormMatmulIO(**ok), "no code object cached")


def test_code_object_row_launcher_refusals():
    rows, cols = 16384, 8192
    r = _object_runtime("fused_residual_rmsnorm", dict(M=rows, N=cols, K=0), ROW)
    ok = dict(x=4096, r=8192, gamma=12288, out=16384, rows=rows, cols=cols, eps=1e-6)
    for missing in ("x", "r", "out"):
        io = rt.ResidualRmsnormIO(**ok)
        setattr(io, missing, None)
        _refused(r, "fused_residual_rmsnorm", (rows, cols, 0), io, "code object: null tensor pointer")
    _refused(r, "fused_residual_rmsnorm", (rows, cols, 0), rt.ResidualRmsnormIO(**dict(ok, cols=4096)),
             "does not match the selected entry")
    _refused(r, "fused_residual_rmsnorm", (rows, cols, 0), rt.ResidualRmsnormIO(**ok), "no code object cached")
    r = _object_runtime("fused_softmax_mask", dict(M=rows, N=cols, K=0), dict(ROW, num_warps=8, unroll=2))
    ok = dict(logits=4096, mask=8192, out=16384, rows=rows, cols=cols)
    for missing in ("logits", "mask", "out"):
        io = rt.SoftmaxMaskIO(**ok)
        setattr(io, missing, None)
        _refused(r, "fused_softmax_mask", (rows, cols, 0), io, "code object: null tensor pointer")
    _refused(r, "fused_softmax_mask", (rows, cols, 0), rt.SoftmaxMaskIO(**ok), "no code object cached")


def test_code_object_attention_launcher_refusals():
    op, mnk = "fused_kv_append_attention", (512, 4096, 128)
    r = _object_runtime(op, dict(M=512, N=4096, K=128), FLASH)
    ok = dict(Q=4096, Kc=8192, Vc=12288, Kn=16384, Vn=20480, O=24576, B=1, H=32, S_q=512, S_cache=3584,
              D=128, cache_capacity=4096, scale=0.088, causal=1)
    for missing in ("Q", "Kc", "Vc", "Kn", "Vn", "O"):
        io = rt.KvAppendAttentionIO(**ok)
        setattr(io, missing, None)
        _refused(r, op, mnk, io, "code object: null tensor pointer")
    _refused(r, op, mnk, rt.KvAppendAttentionIO(**dict(ok, S_cache=3072)), "does not match the selected entry")
    _refused(r, op, mnk, rt.KvAppendAttentionIO(**ok), "no code object cached")
