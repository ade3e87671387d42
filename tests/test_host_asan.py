"""The runtime's host code under AddressSanitizer + UndefinedBehaviorSanitizer
(host code only: the GPU kernels come from the in-tree library, uninstrumented).

The runtime sources (csrc/runtime/*.cpp) are compiled with g++ -fsanitize=
address,undefined and linked with the library's kernel objects (hipcc output,
uninstrumented: the C-ABI and helpers the runtime calls) into two programs:
the C++ API tests (tests/cpp/runtime_test.cpp) and a mutation fuzzer of the
tuning-cache parser and the CLI's .npy reader (tests/cpp/parser_fuzz.cpp).  The sanitizers then see
every parse, cache and launcher-argument path these programs drive."""
from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
RUNTIME = sorted((ROOT / "polykernel_amd" / "csrc" / "runtime").glob("*.cpp"))
FLAGS = ["-std=c++20", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
         "-fno-sanitize-recover=undefined", "-D__HIP_PLATFORM_AMD__", "-I", str(ROOT / "include"),
         "-I", "/opt/rocm/include"]


@pytest.fixture(scope="module")
def instrumented(tmp_path_factory):
    """The runtime's host sources compiled once with the sanitizers, and the
    library's kernel objects (polykernel_amd/_build/*.o from hipcc, not
    instrumented) that define the C-ABI and the helpers the runtime calls."""
    from concurrent.futures import ThreadPoolExecutor

    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("no g++")
    kernels = sorted(p for p in (ROOT / "polykernel_amd" / "_build").glob("*.o") if not p.name.endswith(".host.o"))
    assert kernels, "build the library first (python -m polykernel_amd.build)"
    out = tmp_path_factory.mktemp("asan")

    def one(src):
        o = out / (src.stem + ".o")
        r = subprocess.run([cxx, *FLAGS, "-c", str(src), "-o", str(o)], capture_output=True, text=True, timeout=600)
        return o, r

    with ThreadPoolExecutor(max_workers=min(8, len(RUNTIME))) as ex:
        built = list(ex.map(one, RUNTIME))
    for o, r in built:
        assert r.returncode == 0, r.stderr[-4000:]
    return [o for o, _ in built], kernels, out


def _build(instrumented, main: Path, name: str) -> Path:
    objs, kernels, out = instrumented
    exe = out / name
    r = subprocess.run([shutil.which("g++"), *FLAGS, str(main), *map(str, objs), *map(str, kernels), "-o", str(exe),
                        "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib"],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-4000:]
    return exe


def _env():
    env = dict(os.environ)
    # the HIP runtime keeps allocations until exit; leaks are not what this checks
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1"
    return env


def test_runtime_api_under_sanitizers(instrumented):
    exe = _build(instrumented, ROOT / "tests" / "cpp" / "runtime_test.cpp", "runtime_test_asan")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=_env())
    assert r.returncode == 0 and "ALL PASSED" in r.stdout, (r.stdout + r.stderr)[-4000:]


def test_tuning_parser_fuzz_under_sanitizers(instrumented):
    from polykernel_amd import runtime as rt

    exe = _build(instrumented, ROOT / "tests" / "cpp" / "parser_fuzz.cpp", "parser_fuzz")
    scratch = exe.parent / "scratch"
    scratch.mkdir(exist_ok=True)
    r = subprocess.run([str(exe), str(rt.TUNING_FILE), "4000", "20261202", str(scratch)], capture_output=True,
                       text=True, timeout=300, env=_env())
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    cases, accepted, refused, npy_read, npy_refused = (int(x) for x in r.stdout.split()[1::2])
    assert cases == 4000 and refused > 1000 and accepted > 0, r.stdout
    assert npy_read + npy_refused == 1000 and npy_refused > 100, r.stdout
