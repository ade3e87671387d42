"""Build the gfx950 kernel library in-tree.

    python -m polykernel_amd.build          # -> polykernel_amd/libpolykernel_amd.so

Every csrc/*.hip file is compiled by hipcc for gfx950 only (no CUDA, no other
targets), every csrc/runtime/*.cpp file (host-only: tuning cache, kernel cache,
runtime, autotuner) by g++ as C++20, and both are linked into one shared
library exporting the C-ABI of include/polykernel_amd.h and
include/polykernel_amd_runtime.h plus the C++ API of
include/polykernel_amd_runtime.hpp.  Packed-fp32 instruction selection is turned
off (-packed-fp32-ops); fp32 division and square root keep HIP's correctly
rounded defaults (no fast-math).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "libpolykernel_amd.so"
ARCH = "gfx950"

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # fully unroll the GEMM epilogues (256 accumulators per lane): above the
    # default threshold the accumulator array is demoted to scratch memory
    "-mllvm", "-pragma-unroll-threshold=1000000",
    "-Wno-unused-result",
    "-I", str(PKG.parent / "include"),
]


# Host-only runtime (tuning cache, kernel cache, autotuner): plain C++20.
CXX = shutil.which("g++") or "g++"
HOST_FLAGS = [
    "-std=c++20", "-O2", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wextra", "-Wno-unused-parameter",
    "-D__HIP_PLATFORM_AMD__", "-I", "/opt/rocm/include", "-I", str(PKG.parent / "include"),
]


def _compile(src: Path) -> Path:
    out = OBJ / (src.stem + (".o" if src.suffix == ".hip" else ".host.o"))
    if src.suffix == ".cpp":
        cmd = [CXX, *HOST_FLAGS, "-c", str(src), "-o", str(out)]
    else:
        cmd = [HIPCC, *COMMON_FLAGS, "-c", str(src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        msg = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
        raise RuntimeError(f"{Path(cmd[0]).name} failed for {src.name}:\n{msg}")
    return out


def build(verbose: bool = True) -> Path:
    """Compile every kernel source and link libpolykernel_amd.so (always rebuilds)."""
    OBJ.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip")) + sorted((CSRC / "runtime").glob("*.cpp"))
    if not srcs:
        raise RuntimeError(f"no sources under {CSRC}")
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    build_cli()
    if verbose:
        print(f"[polykernel_amd] built {LIB} from {len(srcs)} sources, and {CLI}", flush=True)
    return LIB


CLI = PKG / "bin" / "pk_hip_run"


def build_cli() -> Path:
    """pk_hip_run: the .npy driver of csrc/cli (links the library and HIP)."""
    CLI.parent.mkdir(exist_ok=True)
    tmp = CLI.with_suffix(".tmp")
    cmd = [CXX, *HOST_FLAGS, str(CSRC / "cli" / "hip_run.cpp"), "-o", str(tmp), str(LIB),
           "-L", "/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,$ORIGIN/..", "-Wl,-rpath,/opt/rocm/lib"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"g++ failed for pk_hip_run:\n{res.stderr}")
    os.replace(tmp, CLI)
    return CLI


if __name__ == "__main__":
    build()
    sys.exit(0)
