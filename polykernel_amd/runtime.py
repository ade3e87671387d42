"""Python face of the C++ runtime (include/polykernel_amd_runtime.h).

Mirrors the reference's runtime classes -- KernelCache (tuning entries per gpu
namespace, code-object binaries with FNV-1a hashes, persistence), Runtime
(detect -> select -> serve) -- over the library's C-ABI.  Every method calls
into libpolykernel_amd.so; nothing here re-implements the selection logic.
"""
from __future__ import annotations

import ctypes as C
import json
from dataclasses import dataclass
from typing import Optional

from . import _lib

OPS = (
    "matmul", "fused_matmul_bias_gelu", "fused_matmul_bias_residual",
    "matmul_int8", "matmul_int8_gelu", "matmul_int8_residual",
    "fused_rmsnorm_matmul", "fused_residual_rmsnorm", "fused_softmax_mask",
    "fused_kv_append_attention",
)


def op_dtype(op: str) -> str:
    """dtype of the op's shape key (the runtime's convention)."""
    if op.startswith("matmul_int8"):
        return "int8"
    if op == "fused_softmax_mask":
        return "fp32"
    return "bf16"


@dataclass(frozen=True)
class Shape:
    m: int
    n: int
    k: int
    dtype: str


class RuntimeError_(RuntimeError):
    """A runtime call failed; `code` is the PK_ERR_* status."""

    def __init__(self, what: str, code: int, message: str):
        super().__init__(f"{what}: {message}")
        self.code = code
        self.message = message


def _call(what: str, rc: int) -> None:
    if rc != _lib.PK_OK:
        raise RuntimeError_(what, rc, _lib.last_error())


def _s(x: Optional[str]) -> Optional[bytes]:
    return None if x is None else x.encode()


# ---- argument blocks (struct pk_*_io) -----------------------------------------
P, I, F, SZ = C.c_void_p, C.c_int, C.c_float, C.c_size_t


class MatmulIO(C.Structure):
    _fields_ = [("A", P), ("B", P), ("C", P), ("bias", P), ("residual", P),
                ("M", I), ("N", I), ("K", I), ("stream", P)]


class MatmulInt8IO(C.Structure):
    _fields_ = [("A", P), ("Wq", P), ("scale", P), ("C", P), ("residual", P),
                ("M", I), ("N", I), ("K", I), ("workspace", P), ("workspace_bytes", SZ), ("stream", P)]


class RmsnormMatmulIO(C.Structure):
    _fields_ = [("x", P), ("gamma", P), ("W", P), ("out", P), ("M", I), ("N", I), ("K", I),
                ("eps", F), ("stream", P)]


class ResidualRmsnormIO(C.Structure):
    _fields_ = [("x", P), ("r", P), ("gamma", P), ("out", P), ("rows", I), ("cols", I),
                ("eps", F), ("stream", P)]


class SoftmaxMaskIO(C.Structure):
    _fields_ = [("logits", P), ("mask", P), ("out", P), ("rows", I), ("cols", I), ("stream", P)]


class KvAppendAttentionIO(C.Structure):
    _fields_ = [("Q", P), ("Kc", P), ("Vc", P), ("Kn", P), ("Vn", P), ("O", P),
                ("B", I), ("H", I), ("S_q", I), ("S_cache", I), ("D", I), ("cache_capacity", I),
                ("scale", F), ("causal", I), ("stream", P)]


# ---- free functions -------------------------------------------------------------

def format_key(gpu: str, op: str, m: int, n: int, k: int, dtype: str) -> str:
    _call("pk_format_key", _lib.load().pk_format_key(_s(gpu), _s(op), m, n, k, _s(dtype)))
    return _lib.last_text()


def hash_file(path: str) -> str:
    """FNV-1a 64 of the file's bytes, 16 lower-case hex digits."""
    _call("pk_hash_file", _lib.load().pk_hash_file(_s(str(path))))
    return _lib.last_text()


def passes_correctness_gate(cosine: float, max_rel_err: float, pcc: float, ceiling: float = 1e-2) -> bool:
    return bool(_lib.load().pk_passes_correctness_gate(cosine, max_rel_err, pcc, ceiling))


def rel_ceiling(op: str, k: int) -> float:
    return _lib.load().pk_rel_ceiling(_s(op), k)


def select_best_validated(results) -> Optional[int]:
    """results: sequence of (validated: bool, time_ms: float | None)."""
    n = len(results)
    if n == 0:
        return None
    val = (C.c_int * n)(*[1 if v else 0 for v, _ in results])
    tms = (C.c_double * n)(*[float("nan") if t is None else float(t) for _, t in results])
    i = _lib.load().pk_select_best_validated(val, tms, n)
    return None if i < 0 else i


def candidates(op: str, m: int, n: int, k: int, dtype: Optional[str] = None) -> list:
    """The configurations the gfx950 kernels implement for (op, shape)."""
    _call("pk_config_candidates",
          _lib.load().pk_config_candidates(_s(op), m, n, k, _s(dtype or op_dtype(op))))
    return json.loads(_lib.last_text())


def default_config(op: str, m: int, n: int, k: int) -> Optional[dict]:
    cfg = _lib.Config()
    rc = _lib.load().pk_op_default_config(_s(op), m, n, k, C.byref(cfg))
    if rc == _lib.PK_ERR_UNSUPPORTED:
        return None
    _call("pk_op_default_config", rc)
    return cfg.as_dict()


def autotune(op: str, m: int, n: int, k: int, dtype: Optional[str] = None, **options) -> dict:
    """Correctness-gated sweep on the current GPU: {"entry": ..., "variants": [...]}."""
    opts = json.dumps(options) if options else None
    _call(f"autotune {op}", _lib.load().pk_autotune(_s(op), m, n, k, _s(dtype or op_dtype(op)), _s(opts)))
    return json.loads(_lib.last_text())


# ---- KernelCache / Runtime ------------------------------------------------------------

class KernelCache:
    """(gpu, op, shape) -> validated tuning entry (+ its code object)."""

    def __init__(self):
        self._lib = _lib.load()
        self._h = self._lib.pk_cache_create()
        if not self._h:
            raise MemoryError("pk_cache_create")

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._lib.pk_cache_destroy(h)

    @property
    def handle(self):
        return self._h

    def load_tuning_cache(self, text: str) -> None:
        _call("LoadTuningCache", self._lib.pk_cache_load_tuning(self._h, _s(text)))

    def put(self, entry: dict) -> None:
        _call("Put", self._lib.pk_cache_put(self._h, _s(json.dumps(entry))))

    def __len__(self) -> int:
        return int(self._lib.pk_cache_size(self._h))

    def serialize(self) -> str:
        _call("Serialize", self._lib.pk_cache_serialize(self._h))
        return _lib.last_text()

    def select(self, gpu: str, op: str, m: int, n: int, k: int, dtype: str) -> dict:
        """The validated entry; raises RuntimeError_ (code PK_ERR_NOT_FOUND) otherwise."""
        _call("Select", self._lib.pk_cache_select(self._h, _s(gpu), _s(op), m, n, k, _s(dtype)))
        return json.loads(_lib.last_text())

    def put_binary(self, gpu: str, op: str, m: int, n: int, k: int, dtype: str, so_path: str,
                   kernel_hash: str) -> None:
        _call("PutBinary", self._lib.pk_cache_put_binary(self._h, _s(gpu), _s(op), m, n, k, _s(dtype),
                                                         _s(str(so_path)), _s(kernel_hash)))

    def get_binary(self, gpu: str, op: str, m: int, n: int, k: int, dtype: str) -> Optional[dict]:
        rc = self._lib.pk_cache_get_binary(self._h, _s(gpu), _s(op), m, n, k, _s(dtype))
        if rc == _lib.PK_ERR_NOT_FOUND:
            return None
        _call("GetBinary", rc)
        return json.loads(_lib.last_text())

    def persist(self, cache_dir: str) -> None:
        _call("Persist", self._lib.pk_cache_persist(self._h, _s(str(cache_dir))))

    def load_persisted(self, cache_dir: str) -> None:
        _call("LoadPersisted", self._lib.pk_cache_load_persisted(self._h, _s(str(cache_dir))))

    def invalidate_stale(self) -> int:
        return int(self._lib.pk_cache_invalidate_stale(self._h))


CODE_OBJECTS = 1  # PK_RUNTIME_CODE_OBJECTS


class Runtime:
    """detect -> select -> serve over a KernelCache, with every built-in
    launcher registered.  fixed_arch=None detects the HIP device.  With
    code_objects=True every op is served from the code object the cache holds
    for its entry (emit_code_object), loaded with hipModuleLoad."""

    def __init__(self, cache: KernelCache, fixed_arch: Optional[str] = None, code_objects: bool = False):
        self._lib = _lib.load()
        self._cache = cache  # keep the cache alive for the runtime's lifetime
        self._h = self._lib.pk_runtime_create_ex(cache.handle, _s(fixed_arch), CODE_OBJECTS if code_objects else 0)
        if not self._h:
            raise RuntimeError_("pk_runtime_create", _lib.PK_ERR_INVALID_ARG, _lib.last_error())

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._lib.pk_runtime_destroy(h)

    def resolve(self, op: str, m: int, n: int, k: int, dtype: Optional[str] = None) -> dict:
        _call("Resolve", self._lib.pk_runtime_resolve(self._h, _s(op), m, n, k, _s(dtype or op_dtype(op))))
        return json.loads(_lib.last_text())

    def run(self, op: str, m: int, n: int, k: int, io: C.Structure, dtype: Optional[str] = None) -> None:
        _call(f"Run {op}", self._lib.pk_runtime_run(self._h, _s(op), m, n, k, _s(dtype or op_dtype(op)),
                                                    C.byref(io)))


# ---- emitter --------------------------------------------------------------------------

CSRC_DIR = _lib._PKG / "csrc"


def emit_source(entry: dict) -> str:
    """gfx950 HIP source instantiating a tuned entry's kernel template at its config."""
    _call("emit_source", _lib.load().pk_emit_source(_s(json.dumps(entry))))
    return _lib.last_text()


def emit_code_object(cache: KernelCache, entry: dict, out_dir) -> dict:
    """Compile the entry's code object into out_dir (hipcc --genco, child
    process) and record entry + object in `cache`; returns the binary record."""
    _call("emit_code_object", _lib.load().pk_emit_code_object(cache.handle, _s(json.dumps(entry)),
                                                              _s(str(CSRC_DIR)), _s(str(out_dir))))
    sh = entry["shape"]
    return cache.get_binary(entry["gpu"], entry["op"], sh["M"], sh["N"], sh["K"], sh["dtype"])


# ---- the committed gfx950 tuning cache ----------------------------------------------

TUNING_FILE = _lib._PKG / "tuning" / "gfx950.json"


def default_cache() -> KernelCache:
    """A KernelCache holding the committed gfx950 entries (polykernel_amd/tuning/gfx950.json,
    written by `python -m polykernel_amd.autotune --baseline`)."""
    cache = KernelCache()
    cache.load_tuning_cache(TUNING_FILE.read_text())
    return cache


def default_runtime() -> Runtime:
    """Runtime over default_cache() with the HIP device detector."""
    return Runtime(default_cache())


CODE_OBJECT_DIR = TUNING_FILE.with_suffix(".d")


def code_object_cache(cache_dir=CODE_OBJECT_DIR) -> KernelCache:
    """The persisted cache written by `python -m polykernel_amd.emit` (entries
    plus their code objects); stale code objects are dropped on load."""
    cache = KernelCache()
    cache.load_persisted(cache_dir)
    cache.invalidate_stale()
    return cache
