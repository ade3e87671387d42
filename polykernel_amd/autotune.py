"""Correctness-gated autotuner CLI: sweep the gfx950 variants of an op on the
current GPU and write the winners into a tuning-cache file.

    python -m polykernel_amd.autotune --baseline --out polykernel_amd/tuning/gfx950.json \
        --log polykernel_amd/tuning/gfx950.sweep.jsonl
    python -m polykernel_amd.autotune --op matmul_int8 --shape 16,28672,8192

Each (op, shape) goes through pk_autotune (csrc/runtime/autotune.cpp): every
candidate is compared with a naive device golden and gated (cosine >= 0.999,
pcc >= 0.99, max_rel_err <= the reference's ceiling rule) before it is timed;
the fastest validated variant becomes the entry.  GEMM-class ops are also
gated on the per-element fp32 error model (model_violations must be 0).
--log writes one JSON line per swept variant (config, its metrics, model
violations, validated, median time) -- the record of what each committed
entry passed, since the entry itself keeps only the schema's fields.
Entries are merged into
the output file (last writer wins per (gpu, op, shape)), which is the
tuning-cache document of tuning/schema.json and loads with
runtime.KernelCache.load_tuning_cache -- the default cache of
runtime.default_runtime().
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

from . import runtime as rt

# The shapes of the headline configurations, as (op, M, N, K) in the
# runtime's shape keys (fused_kv_append_attention: S_q, S_kv, D).
BASELINE = [
    ("fused_rmsnorm_matmul", 128, 3072, 768),         # config 1
    ("fused_matmul_bias_gelu", 4096, 16384, 4096),    # config 2, GEMM1
    ("fused_matmul_bias_residual", 4096, 4096, 16384),  # config 2, GEMM2
    ("fused_kv_append_attention", 512, 4096, 128),    # config 3 (B*H = 32)
    ("fused_residual_rmsnorm", 16384, 8192, 0),       # config 4a
    ("fused_softmax_mask", 16384, 8192, 0),           # config 4b
    ("matmul_int8_gelu", 16, 28672, 8192),            # config 5, W1
    ("matmul_int8_residual", 16, 8192, 28672),        # config 5, W2
]


def merge(path: Path, entries: list) -> str:
    """Merge entries into the tuning-cache file at `path` (created if absent)."""
    cache = rt.KernelCache()
    if path.exists():
        cache.load_tuning_cache(path.read_text())
    for e in entries:
        cache.put(e)
    text = cache.serialize()
    path.parent.mkdir(parents=True, exist_ok=True)
    # one entry per line keeps diffs of the committed file readable
    doc = json.loads(text)
    lines = ",\n".join("  " + json.dumps(e, sort_keys=True, separators=(",", ":")) for e in doc["entries"])
    path.write_text('{"version":1,"entries":[\n' + lines + "\n]}\n")
    return text


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--op", choices=rt.OPS)
    ap.add_argument("--shape", help="M,N,K in the op's shape key")
    ap.add_argument("--baseline", action="store_true", help="sweep every headline configuration's shapes")
    ap.add_argument("--out", type=Path, help="tuning-cache file to merge the entries into")
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--rounds", type=int, default=5, help="interleaved timing passes over the gated variants")
    ap.add_argument("--max-variants", type=int, default=None)
    ap.add_argument("--log", type=Path, help="write every swept variant's gate outcome here (JSON lines)")
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args(argv)
    if args.baseline == bool(args.op):
        ap.error("give either --baseline or --op/--shape")
    jobs = BASELINE if args.baseline else [(args.op, *map(int, args.shape.split(",")))]
    opts = dict(iters=args.iters, warmup=args.warmup, rounds=args.rounds, verbose=args.verbose)
    if args.max_variants:
        opts["max_variants"] = args.max_variants
    entries, failed, log = [], 0, []
    for op, m, n, k in jobs:
        t0 = time.time()
        res = rt.autotune(op, m, n, k, **opts)
        e = res["entry"]
        ok = sum(v["validated"] for v in res["variants"])
        print(f"[autotune] {op} M={m} N={n} K={k}: {len(res['variants'])} variants, {ok} validated, "
              f"best {e['best']} {e['time_ms']} ms, validated={e['validated']} ({time.time() - t0:.1f} s)",
              flush=True)
        failed += not e["validated"]
        entries.append(e)
        for v in res["variants"]:
            log.append({"op": op, "shape": [m, n, k], "selected": v["config"] == e["best"], **v})
    if args.out:
        merge(args.out, entries)
        print(f"[autotune] wrote {len(entries)} entries to {args.out}", flush=True)
    if args.log:
        args.log.parent.mkdir(parents=True, exist_ok=True)
        args.log.write_text("".join(json.dumps(r, sort_keys=True) + "\n" for r in log))
        print(f"[autotune] wrote {len(log)} variant records to {args.log}", flush=True)
    return 1 if failed else 0


if __name__ == "__main__":
    sys.exit(main())
