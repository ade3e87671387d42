"""Emit the gfx950 code objects of a tuning cache's entries.

    python -m polykernel_amd.emit                      # committed cache -> polykernel_amd/tuning/gfx950.d
    python -m polykernel_amd.emit --cache X.json --out DIR

For every entry of the cache (GEMM family, RMSNorm -> MatMul, residual +
RMSNorm, masked softmax, int8, attention) the emitter
(csrc/runtime/codegen.cpp) writes a HIP source that instantiates the kernel
template (gemm_kernels.hpp, rowwise_kernels.hpp, int8_stream.hpp,
attention_kernels.hpp) at the entry's configuration, compiles it for gfx950
with hipcc --genco (no GPU needed) and
records the code object's path and FNV-1a hash beside the entry.  The result
is persisted as DIR/tuning_db.json + DIR/binaries.json (the KernelCache
persistence format); runtime.Runtime(..., code_objects=True) over
runtime.code_object_cache(DIR) serves those ops from the code objects.
"""
from __future__ import annotations

import argparse
import json
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

from . import runtime as rt

DEFAULT_OUT = rt.TUNING_FILE.with_suffix(".d")
EMIT_OPS = ("matmul", "fused_matmul_bias_gelu", "fused_matmul_bias_residual", "fused_rmsnorm_matmul",
            "fused_residual_rmsnorm", "fused_softmax_mask",
            "matmul_int8", "matmul_int8_gelu", "matmul_int8_residual", "fused_kv_append_attention")


def emit(cache_file: Path = rt.TUNING_FILE, out_dir: Path = DEFAULT_OUT, verbose: bool = True) -> int:
    """Emit every entry of cache_file into out_dir; returns the count."""
    doc = json.loads(Path(cache_file).read_text())
    entries = [e for e in doc["entries"] if e["op"] in EMIT_OPS and e["validated"]]
    cache = rt.KernelCache()
    cache.load_tuning_cache(Path(cache_file).read_text())
    return _emit_entries(entries, cache, Path(out_dir), verbose)


# Conformance set: every kernel template the emitter instantiates, at small
# shapes, so that the GPU tests can compare each emitted object with the
# linked kernel at the same configuration.  These entries are not tuned
# (scored_by "model", no time); they live in their own cache directory and
# are never served by the default runtimes.
CONFORMANCE_OUT = rt.TUNING_FILE.with_name("gfx950.conformance.d")
GEMM_SHAPE = (200, 264, 256)  # ragged M and N tiles for every tile size
INT8_SHAPE = (24, 1040, 1024)
ATT_SQ, ATT_SCACHE, ATT_HEAD_DIMS = 200, 256, (64, 128, 96, 256, 512, 300)
# row ops: 37 rows (ragged for four rows per workgroup); the widths reach
# every vector kernel (one wave per row with 1/2/4/8 vectors per lane, four
# waves per row with 2/4/8, eight with 1/2/4/8/16, sixteen with 4/8 and the
# packed-bf16 16x16) and the generic kernel (cols % 8 != 0, or more than
# 131072 columns)
ROW_ROWS, ROW_COLS = 37, (512, 1024, 2048, 4096, 8192, 16384, 32768, 65536, 70000, 131072, 140000, 1000, 999)
# RMSNorm -> MatMul: the whole-K panel (ragged M) and the RMSNorm-into-
# workspace path followed by a GEMM (K 1536 and 2048); at K 64 the panel
# (64 x 256), and the 64-deep GEMM configs whose block_k equals K: N % 8 != 0
# (no panel) and more than 256 panel tiles (33 x 8)
PANEL_SHAPES = ((40, 136, 768), (64, 256, 1536), (72, 264, 2048), (64, 256, 64), (40, 1001, 64), (1056, 512, 64))


def conformance_entries() -> list:
    out = []

    def entry(op, shape, dtype, cfg):
        M, N, K = shape
        return {"gpu": "gfx950", "op": op, "shape": {"M": M, "N": N, "K": K, "dtype": dtype}, "best": cfg,
                "scored_by": "model", "time_ms": None, "validated": True,
                "correctness": {"cosine": 1.0, "max_rel_err": 0.0, "pcc": 1.0}}

    for op in ("matmul", "fused_matmul_bias_gelu", "fused_matmul_bias_residual"):
        for cfg in rt.candidates(op, *GEMM_SHAPE):
            out.append(entry(op, GEMM_SHAPE, "bf16", cfg))
    # attention shape key (S_q, S_cache + S_q, D); S_cache 256 sits on the
    # key step of both flash tile shapes, so the fused append applies
    for D in ATT_HEAD_DIMS:
        shape = (ATT_SQ, ATT_SCACHE + ATT_SQ, D)
        for cfg in rt.candidates("fused_kv_append_attention", *shape):
            out.append(entry("fused_kv_append_attention", shape, "bf16", cfg))
    for op, dtype in (("fused_residual_rmsnorm", "bf16"), ("fused_softmax_mask", "fp32")):
        for cols in ROW_COLS:
            for cfg in rt.candidates(op, ROW_ROWS, cols, 0):
                out.append(entry(op, (ROW_ROWS, cols, 0), dtype, cfg))
    for shape in PANEL_SHAPES:
        for cfg in rt.candidates("fused_rmsnorm_matmul", *shape):
            out.append(entry("fused_rmsnorm_matmul", shape, "bf16", cfg))
    cands = rt.candidates("matmul_int8_residual", *INT8_SHAPE)
    split = next(c for c in cands if c["block_k"] < INT8_SHAPE[2])
    for op in ("matmul_int8", "matmul_int8_gelu", "matmul_int8_residual"):
        out.append(entry(op, INT8_SHAPE, "int8", cands[0]))
        out.append(entry(op, INT8_SHAPE, "int8", split))
    return out


def emit_conformance(out_dir: Path = CONFORMANCE_OUT, verbose: bool = False) -> int:
    """Emit the conformance set into out_dir/objects and list every (entry,
    code object, hash) in out_dir/manifest.json (a cache holds one entry per
    (op, shape), so the GPU test builds one cache per manifest line)."""
    done = _emit_entries(conformance_entries(), None, Path(out_dir), verbose)
    manifest = [{"entry": e, "so_path": b["so_path"], "kernel_hash": b["kernel_hash"]} for e, b in done]
    (Path(out_dir) / "manifest.json").write_text(json.dumps(manifest, indent=1) + "\n")
    return len(done)


def _emit_entries(entries, cache, out_dir: Path, verbose: bool):
    """Emit each entry's code object; with a cache, record the objects in it
    and persist it to out_dir (returns the count), else return the list of
    (entry, binary) pairs."""
    objects = Path(out_dir) / "objects"
    # objects of an earlier emission (other configs, older file names) go
    if objects.is_dir():
        for f in objects.iterdir():
            if f.suffix in (".hip", ".hsaco", ".log"):
                f.unlink()

    # compile in parallel (each a hipcc child process), record in order
    def one(e):
        scratch = rt.KernelCache()
        return e, rt.emit_code_object(scratch, e, objects)

    with ThreadPoolExecutor(max_workers=max(1, min(8, len(entries)))) as ex:
        done = list(ex.map(one, entries))
    if cache is None:
        return done
    for e, binary in done:
        sh = e["shape"]
        cache.put_binary(e["gpu"], e["op"], sh["M"], sh["N"], sh["K"], sh["dtype"], binary["so_path"],
                         binary["kernel_hash"])
        if verbose:
            print(f"[emit] {e['op']} M={sh['M']} N={sh['N']} K={sh['K']} -> {binary['so_path']} "
                  f"({binary['kernel_hash']})", flush=True)
    cache.persist(out_dir)
    return len(done)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--cache", type=Path, default=rt.TUNING_FILE)
    ap.add_argument("--out", type=Path, default=DEFAULT_OUT)
    args = ap.parse_args(argv)
    n = emit(args.cache, args.out)
    print(f"[emit] {n} code objects, cache persisted to {args.out}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
