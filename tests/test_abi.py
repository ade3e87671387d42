"""The built library loads and exports every entry point include/*.h declares
(CPU only: symbols are resolved, nothing is launched)."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))
_DECL = re.compile(r"PK_API\s+[^;{]*?\b([A-Za-z_][A-Za-z0-9_]*)\s*\(", re.S)


def _header_text(h: Path) -> str:
    """Declarations only: comments and preprocessor lines removed."""
    text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
    return "\n".join(l for l in text.splitlines() if not l.lstrip().startswith("#"))


def declared_symbols():
    names = []
    for h in HEADERS:
        names += _DECL.findall(_header_text(h))
    return sorted(set(names))


def test_headers_declare_entry_points():
    names = declared_symbols()
    # the reference's launch_* names and the runtime C-ABI are both there
    for must in ("launch_matmul", "launch_fused_rmsnorm_matmul", "launch_matmul_int8",
                 "launch_attention_prefill", "pk_cache_select", "pk_runtime_run", "pk_autotune"):
        assert must in names
    assert len(names) > 60


@pytest.mark.parametrize("name", declared_symbols())
def test_symbol_exported(name):
    from polykernel_amd import _lib

    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    assert hasattr(lib, name), f"{name} declared in include/ but not exported by {_lib.LIB_PATH.name}"


def test_ctypes_signatures_cover_headers():
    """Every declared entry point has a ctypes signature (argument count
    checked by the declaration's comma count)."""
    from polykernel_amd import _lib

    missing = [n for n in declared_symbols() if n not in _lib.SIGNATURES]
    assert not missing, f"no ctypes signature for {missing}"
    text = "".join(_header_text(h) for h in HEADERS)
    for name, (_, args) in _lib.SIGNATURES.items():
        m = re.search(r"PK_API\s+[^;{]*?\b" + name + r"\s*\(([^)]*)\)", text, re.S)
        assert m, name
        params = m.group(1).strip()
        n = 0 if params in ("", "void") else params.count(",") + 1
        assert n == len(args), f"{name}: header has {n} parameters, ctypes {len(args)}"
