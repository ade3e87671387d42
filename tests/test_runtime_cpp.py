"""Build tests/cpp/runtime_test.cpp against the in-tree library and run it
(the C++ API of include/polykernel_amd_runtime.hpp; no GPU needed)."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def test_cpp_runtime_api(tmp_path):
    from polykernel_amd import _lib

    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("no g++")
    lib = _lib.LIB_PATH
    assert lib.exists(), "build the library first (python -m polykernel_amd.build)"
    exe = tmp_path / "runtime_test"
    build = subprocess.run(
        [cxx, "-std=c++20", "-O1", "-Wall", "-D__HIP_PLATFORM_AMD__", "-I", str(ROOT / "include"),
         "-I", "/opt/rocm/include", str(ROOT / "tests" / "cpp" / "runtime_test.cpp"),
         "-o", str(exe), str(lib), f"-Wl,-rpath,{lib.parent}"],
        capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0 and "ALL PASSED" in run.stdout, run.stdout + run.stderr
