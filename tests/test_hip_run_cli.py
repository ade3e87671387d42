"""pk_hip_run's .npy bridge on the CPU ('info' and 'roundtrip' need no GPU):
bf16 '<V2', int8 '|i1', fp32 '<f4'; NumPy reads what it writes; the header is
the reference writer's (kernels/cpu/npy_io.cpp:127-171); bad input is an
error, never a crash."""
from __future__ import annotations

import subprocess

import numpy as np
import pytest

from polykernel_amd import build as pkbuild


def run(*args):
    if not pkbuild.CLI.exists():
        pytest.skip("pk_hip_run not built")
    return subprocess.run([str(pkbuild.CLI), *map(str, args)], capture_output=True, text=True, timeout=60)


def test_roundtrip_bf16_matches_reference_header(tmp_path):
    bits = np.arange(6, dtype=np.uint16).reshape(2, 3) * 0x1111
    src = tmp_path / "in.npy"
    np.save(src, bits.view("V2"))  # NumPy writes '|V2'
    out = tmp_path / "out.npy"
    r = run("roundtrip", src, out)
    assert r.returncode == 0, r.stderr
    data = out.read_bytes()
    dict_ = b"{'descr': '<V2', 'fortran_order': False, 'shape': (2, 3), }"
    assert data[:10] == b"\x93NUMPY\x01\x00" + (len(data) - 10 - 12).to_bytes(2, "little")
    header = data[10:10 + int.from_bytes(data[8:10], "little")]
    assert header.startswith(dict_) and header.endswith(b"\n") and (10 + len(header)) % 64 == 0
    assert set(header[len(dict_):-1]) <= {ord(" ")}
    back = np.load(out)
    assert back.dtype.itemsize == 2 and np.array_equal(back.view(np.uint16), bits)


@pytest.mark.parametrize("arr,descr", [(np.arange(-5, 7, dtype=np.int8).reshape(3, 4), "|i1"),
                                       (np.linspace(-1, 1, 10, dtype=np.float32), "<f4"),
                                       (np.zeros((0, 4), dtype=np.float32), "<f4")])
def test_roundtrip_int8_fp32(tmp_path, arr, descr):
    src, out = tmp_path / "a.npy", tmp_path / "b.npy"
    np.save(src, arr)
    r = run("info", src)
    assert r.returncode == 0 and f"descr={descr}" in r.stdout, r.stdout + r.stderr
    assert run("roundtrip", src, out).returncode == 0
    back = np.load(out)
    assert back.dtype == arr.dtype and back.shape == arr.shape and np.array_equal(back, arr)


def test_shapes_in_reference_repr(tmp_path):
    for shape, text in [((7,), "(7,)"), ((), "()"), ((1, 2, 3, 4), "(1, 2, 3, 4)")]:
        src = tmp_path / "s.npy"
        np.save(src, np.zeros(shape, dtype=np.float32))
        r = run("info", src)
        assert f"shape={text}" in r.stdout, r.stdout


def test_bad_inputs_are_errors(tmp_path):
    f8 = tmp_path / "f8.npy"
    np.save(f8, np.zeros(4, dtype=np.float64))
    r = run("info", f8)
    assert r.returncode == 1 and "unsupported dtype '<f8'" in r.stderr
    fortran = tmp_path / "f.npy"
    np.save(fortran, np.asfortranarray(np.zeros((3, 4), dtype=np.float32)))
    r = run("info", fortran)
    assert r.returncode == 1 and "Fortran" in r.stderr
    junk = tmp_path / "junk.npy"
    junk.write_bytes(b"not numpy at all")
    assert run("info", junk).returncode == 1
    trunc = tmp_path / "t.npy"
    np.save(trunc, np.zeros(100, dtype=np.float32))
    trunc.write_bytes(trunc.read_bytes()[:-8])
    r = run("info", trunc)
    assert r.returncode == 1 and "truncated" in r.stderr
    assert run("matmul", "a.npy").returncode == 2          # wrong arity: usage
    assert run("frobnicate").returncode == 2               # unknown op
    assert run("softmax", "a", "b", "--nope", "1").returncode == 2


def _npy_with_header(path, header: str, payload: bytes = bytes(16)):
    h = header.encode()
    h = h + b" " * (64 - (10 + len(h) + 1) % 64) + b"\n"
    path.write_bytes(b"\x93NUMPY\x01\x00" + len(h).to_bytes(2, "little") + h + payload)


@pytest.mark.parametrize("shape,msg", [("(99999999999999999999,)", "is too large"),
                                       ("(4000000000, 4000000000, 4000000000)", "is too large"),
                                       ("(400000000000, 4)", "truncated .npy payload"),
                                       ("(5, 4)", "truncated .npy payload")])
def test_oversized_or_truncated_payload_is_refused_before_allocating(tmp_path, shape, msg):
    """A header whose shape overflows, or declares more bytes than the file
    holds, is an error with a message; nothing is allocated for it."""
    f = tmp_path / "bad.npy"
    _npy_with_header(f, "{'descr': '<f4', 'fortran_order': False, 'shape': %s, }" % shape)
    r = run("roundtrip", f, tmp_path / "out.npy")
    assert r.returncode == 1 and msg in r.stderr, r.stderr
