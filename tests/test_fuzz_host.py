"""Mutation fuzzing of the host-side parsers that read files a user hands the
runtime: the tuning-cache JSON (KernelCache::LoadTuningCache, the reference's
lib/Autotune/TuningCache.cpp format), the persisted cache directory
(tuning_db.json + binaries.json, KernelCache::LoadPersisted) and pk_hip_run's
.npy reader.  Every mutated input must load or be refused with an error code
and message -- never crash or hang the process.  The parsers run in child
processes so that a crash is reported as this test's failure with its seed.
"""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from polykernel_amd import build as pkbuild

ROOT = Path(__file__).resolve().parents[1]

# Mutations of a byte string: delete, insert, overwrite with a JSON-significant
# byte, or truncate, 1-8 of them per case (seeded, so a failure names its case).
MUTATE = r'''
import random
SIG = b'{}[]",:0123456789.-+eE truefalsn\\u\x00\xff\xc3'
def mutate(data, rng):
    s = bytearray(data)
    for _ in range(rng.randint(1, 8)):
        op = rng.randrange(4)
        pos = rng.randrange(len(s) + 1)
        if op == 0 and s:
            del s[min(pos, len(s) - 1)]
        elif op == 1:
            s.insert(pos, rng.randrange(256))
        elif op == 2 and s:
            s[min(pos, len(s) - 1)] = SIG[rng.randrange(len(SIG))]
        else:
            s = s[:pos]
    return bytes(s)
'''


def _child(code: str, timeout: int = 240) -> str:
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=timeout,
                       cwd=str(ROOT))
    assert r.returncode == 0, f"rc={r.returncode}\n{r.stdout[-2000:]}\n{r.stderr[-2000:]}"
    return r.stdout


def test_tuning_cache_json_survives_mutations():
    out = _child(MUTATE + r'''
import ctypes, random, sys
sys.path.insert(0, ".")
from polykernel_amd import _lib, runtime as rt
lib = _lib.load()
base = rt.TUNING_FILE.read_bytes()
ok = err = 0
for case in range(3000):
    print("case", case, flush=True) if case % 1000 == 0 else None
    c = rt.KernelCache()
    rc = lib.pk_cache_load_tuning(c._h, mutate(base, random.Random(case)))
    if rc == 0:
        ok += 1
    else:
        assert rc < 0 and _lib.last_error(), (case, rc)
        err += 1
print("result", ok, err)
''')
    ok, err = map(int, out.split("result")[1].split())
    assert ok + err == 3000 and err > 1000 and ok > 0, (ok, err)


def test_persisted_cache_dir_survives_mutations(tmp_path):
    src = tmp_path / "src"
    out = _child(MUTATE + rf'''
import json, random, sys
from pathlib import Path
sys.path.insert(0, ".")
from polykernel_amd import _lib, runtime as rt
src = Path({str(src)!r})
cache = rt.KernelCache()
cache.load_tuning_cache(rt.TUNING_FILE.read_text())
doc = json.loads(rt.TUNING_FILE.read_text())
e = doc["entries"][0]
sh = e["shape"]
obj = src / "x.hsaco"
src.mkdir(parents=True)
obj.write_bytes(b"\x7fELF" + bytes(60))
cache.put_binary(e["gpu"], e["op"], sh["M"], sh["N"], sh["K"], sh["dtype"], str(obj), rt.hash_file(obj))
cache.persist(src)
files = {{n: (src / n).read_bytes() for n in ("tuning_db.json", "binaries.json")}}
ok = err = 0
for case in range(600):
    rng = random.Random(case)
    d = src.parent / f"case{{case % 4}}"
    d.mkdir(exist_ok=True)
    target = "binaries.json" if case % 2 else "tuning_db.json"
    for n, data in files.items():
        (d / n).write_bytes(mutate(data, rng) if n == target else data)
    c = rt.KernelCache()
    rc = _lib.load().pk_cache_load_persisted(c._h, str(d).encode())
    if rc == 0:
        ok += 1
    else:
        assert rc < 0 and _lib.last_error(), (case, rc)
        err += 1
print("result", ok, err)
''')
    ok, err = map(int, out.split("result")[1].split())
    assert ok + err == 600 and err > 100, (ok, err)


@pytest.mark.parametrize("arr", [np.arange(24, dtype=np.uint16).reshape(4, 6).view("V2"),
                                 np.arange(-6, 6, dtype=np.int8).reshape(3, 4),
                                 np.linspace(-1, 1, 8, dtype=np.float32).reshape(2, 4)])
def test_npy_reader_survives_mutations(tmp_path, arr):
    """Header and body mutations of a valid '<V2' / '|i1' / '<f4' file: pk_hip_run
    roundtrip exits 0 (a file that is still valid) or 1 with a message on
    stderr, never by a signal."""
    if not pkbuild.CLI.exists():
        pytest.skip("pk_hip_run not built")
    import random

    src = tmp_path / "valid.npy"
    np.save(src, arr)
    data = src.read_bytes()
    ns = {}
    exec(MUTATE, ns)
    outcomes = {0: 0, 1: 0}
    for case in range(100):
        f = tmp_path / "case.npy"
        f.write_bytes(ns["mutate"](data, random.Random(case)))
        r = subprocess.run([str(pkbuild.CLI), "roundtrip", str(f), str(tmp_path / "out.npy")], capture_output=True,
                           text=True, timeout=20)
        assert r.returncode in (0, 1), (case, r.returncode, r.stderr[-500:])
        if r.returncode == 1:
            assert "error" in r.stderr, (case, r.stderr)
        outcomes[r.returncode] += 1
    assert outcomes[1] > 0
