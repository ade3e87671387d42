"""Emit the gfx950 code objects of a tuning cache's int8 entries.

    python -m polykernel_amd.emit                      # committed cache -> polykernel_amd/tuning/gfx950.d
    python -m polykernel_amd.emit --cache X.json --out DIR

For every int8 entry of the cache the emitter (csrc/runtime/codegen.cpp)
writes a HIP source that instantiates the streaming kernel at the entry's
configuration, compiles it for gfx950 with hipcc --genco (no GPU needed) and
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
INT8_OPS = ("matmul_int8", "matmul_int8_gelu", "matmul_int8_residual")


def emit(cache_file: Path = rt.TUNING_FILE, out_dir: Path = DEFAULT_OUT, verbose: bool = True) -> int:
    """Emit every int8 entry of cache_file into out_dir; returns the count."""
    doc = json.loads(Path(cache_file).read_text())
    entries = [e for e in doc["entries"] if e["op"] in INT8_OPS and e["validated"]]
    cache = rt.KernelCache()
    cache.load_tuning_cache(Path(cache_file).read_text())
    objects = Path(out_dir) / "objects"

    # compile in parallel (each a hipcc child process), record in order
    def one(e):
        scratch = rt.KernelCache()
        return e, rt.emit_code_object(scratch, e, objects)

    with ThreadPoolExecutor(max_workers=max(1, min(8, len(entries)))) as ex:
        done = list(ex.map(one, entries))
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
