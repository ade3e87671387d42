"""ctypes binding of libpolykernel_amd.so (the C-ABI of include/polykernel_amd.h
and include/polykernel_amd_runtime.h).

The library is loaded from the package directory only.  If it is missing the
import fails loudly -- there is no CPU fallback for any kernel.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

_PKG = Path(__file__).resolve().parent
LIB_PATH = _PKG / "libpolykernel_amd.so"

PK_OK = 0
PK_ERR_INVALID_ARG = -1
PK_ERR_LAUNCH = -2
PK_ERR_WORKSPACE = -3
PK_ERR_NO_DEVICE = -4
PK_ERR_UNSUPPORTED = -5
PK_ERR_HIP = -6
PK_ERR_NOT_FOUND = -7


class PolyKernelError(RuntimeError):
    """A launcher returned a non-zero status; carries the library's message."""

    def __init__(self, name: str, code: int, message: str):
        super().__init__(f"{name} failed with status {code}: {message}")
        self.code = code
        self.message = message


class Config(C.Structure):
    """struct pk_config (include/polykernel_amd.h): one kernel configuration in
    the tuning-cache vocabulary; 0 in a request means "any"."""

    _fields_ = [("block_m", C.c_int), ("block_n", C.c_int), ("block_k", C.c_int),
                ("num_warps", C.c_int), ("vector_width", C.c_int), ("unroll", C.c_int),
                ("shared_memory_stages", C.c_int)]

    def as_dict(self) -> dict:
        return {f: getattr(self, f) for f, _ in self._fields_}


P = C.c_void_p
I = C.c_int
F = C.c_float
SZ = C.c_size_t
U64 = C.c_uint64
I64 = C.c_int64
D = C.c_double
LL = C.c_longlong

# name -> (restype, argtypes); mirrors include/polykernel_amd.h
SIGNATURES = {
    "pk_version": (C.c_char_p, []),
    "pk_last_error": (C.c_char_p, []),
    "pk_init": (I, []),
    "pk_device_arch": (I, [I, C.c_char_p, I]),
    "pk_parse_gcn_arch_name": (I, [C.c_char_p, C.c_char_p, I]),
    "pk_check_bf16_conversion": (I, [C.POINTER(C.c_ulonglong)]),
    "pk_check_gelu_pairs": (I, [C.POINTER(C.c_ulonglong)]),
    "pk_check_row_division": (I, [P, I, C.POINTER(C.c_ulonglong)]),
    "launch_rmsnorm": (I, [P, P, P, I, I, F, P]),
    "launch_gelu": (I, [P, P, I, P]),
    "launch_matmul": (I, [P, P, P, I, I, I, P]),
    "launch_softmax": (I, [P, P, I, I, P]),
    "launch_fused_rmsnorm_matmul": (I, [P, P, P, I, I, I, F, P]),
    "launch_fused_matmul_bias_gelu": (I, [P, P, P, P, I, I, I, P]),
    "launch_attention_prefill": (I, [P, P, P, P, I, I, I, I, I, F, I, P]),
    "launch_kv_cache_update": (I, [P, P, P, I, I, I, I, I, P]),
    "launch_matmul_int8": (I, [P, P, P, P, I, I, I, P]),
    "launch_matmul_int8_noalloc": (I, [P, P, P, P, I, I, I, P]),
    "launch_fused_residual_rmsnorm": (I, [P, P, P, P, I, I, F, P]),
    "launch_fused_softmax_mask": (I, [P, P, P, I, I, P]),
    "launch_fused_rmsnorm_matmul_gamma": (I, [P, P, P, P, I, I, I, F, P]),
    "launch_fused_matmul_bias_residual": (I, [P, P, P, P, P, I, I, I, P]),
    "launch_fused_kv_append_attention": (I, [P, P, P, P, P, P, I, I, I, I, I, I, F, I, P]),
    "pk_fused_kv_append_attention_config": (I, [P, P, P, P, P, P, I, I, I, I, I, I, F, I, C.POINTER(Config), P]),
    "pk_fused_residual_rmsnorm_config": (I, [P, P, P, P, I, I, F, C.POINTER(Config), P]),
    "pk_fused_softmax_mask_config": (I, [P, P, P, I, I, C.POINTER(Config), P]),
    "launch_quantize_int8_per_channel": (I, [P, P, P, I, I, P]),
    "pk_mlp_block_workspace_size": (SZ, [I, I, I]),
    "launch_mlp_block": (I, [P, P, P, P, P, P, P, I, I, I, F, P, SZ, P]),
    "pk_decode_mlp_int8_workspace_size": (SZ, [I, I, I]),
    "launch_decode_mlp_int8": (I, [P, P, P, P, P, P, I, I, I, P, SZ, P]),
    "pk_gemm_ex": (I, [I, P, P, P, P, P, I, I, I, I, P]),
    "pk_int8_default_config": (I, [I, I, I, C.POINTER(Config)]),
    "pk_matmul_int8_ex": (I, [I, P, P, P, P, P, I, I, I, C.POINTER(Config), P, SZ, P]),
    "pk_gemm_config_ex": (I, [I, P, P, P, P, P, I, I, I, C.POINTER(Config), P]),
    "pk_op_configs": (I, [C.c_char_p, LL, LL, LL, C.POINTER(Config), I]),
    "pk_op_default_config": (I, [C.c_char_p, LL, LL, LL, C.POINTER(Config)]),
    "pk_naive_matmul": (I, [I, P, P, P, P, P, I, I, I, P]),
    "pk_naive_matmul_int8": (I, [I, P, P, P, P, P, I, I, I, P]),
    "pk_naive_rmsnorm": (I, [P, P, P, P, I, I, F, P]),
    "pk_naive_softmax_mask": (I, [P, P, P, I, I, P]),
    "pk_naive_attention": (I, [P, P, P, P, I, I, I, I, I, F, I, P]),
    "pk_gate_matmul": (I, [I, P, P, P, P, P, I, I, I, D, C.POINTER(C.c_ulonglong), P]),
    "pk_gate_matmul_int8": (I, [I, P, P, P, P, P, I, I, I, C.POINTER(C.c_ulonglong), P]),
    "pk_compare_bf16": (I, [P, P, LL, C.POINTER(D), P]),
    # runtime layer (include/polykernel_amd_runtime.h)
    "pk_last_text": (C.c_char_p, []),
    "pk_cache_create": (P, []),
    "pk_cache_destroy": (None, [P]),
    "pk_cache_load_tuning": (I, [P, C.c_char_p]),
    "pk_cache_put": (I, [P, C.c_char_p]),
    "pk_cache_size": (LL, [P]),
    "pk_cache_serialize": (I, [P]),
    "pk_cache_select": (I, [P, C.c_char_p, C.c_char_p, LL, LL, LL, C.c_char_p]),
    "pk_cache_put_binary": (I, [P, C.c_char_p, C.c_char_p, LL, LL, LL, C.c_char_p, C.c_char_p, C.c_char_p]),
    "pk_cache_get_binary": (I, [P, C.c_char_p, C.c_char_p, LL, LL, LL, C.c_char_p]),
    "pk_cache_persist": (I, [P, C.c_char_p]),
    "pk_cache_load_persisted": (I, [P, C.c_char_p]),
    "pk_cache_invalidate_stale": (LL, [P]),
    "pk_hash_file": (I, [C.c_char_p]),
    "pk_format_key": (I, [C.c_char_p, C.c_char_p, LL, LL, LL, C.c_char_p]),
    "pk_passes_correctness_gate": (I, [D, D, D, D]),
    "pk_rel_ceiling": (D, [C.c_char_p, LL]),
    "pk_select_best_validated": (I, [C.POINTER(I), C.POINTER(D), I]),
    "pk_config_candidates": (I, [C.c_char_p, LL, LL, LL, C.c_char_p]),
    "pk_runtime_create": (P, [P, C.c_char_p]),
    "pk_runtime_create_ex": (P, [P, C.c_char_p, I]),
    "pk_emit_source": (I, [C.c_char_p]),
    "pk_emit_code_object": (I, [P, C.c_char_p, C.c_char_p, C.c_char_p]),
    "pk_gelu_table": (I, [C.POINTER(P)]),
    "pk_probe_invalid_launch": (I, [C.POINTER(I), C.POINTER(I)]),
    "pk_probe_empty_launch": (I, [I, I, I, P]),
    "pk_library_workspace": (I, [SZ, P, C.POINTER(P)]),
    "pk_release_workspace": (I, [P]),
    "pk_runtime_destroy": (None, [P]),
    "pk_runtime_resolve": (I, [P, C.c_char_p, LL, LL, LL, C.c_char_p]),
    "pk_runtime_run": (I, [P, C.c_char_p, LL, LL, LL, C.c_char_p, P]),
    "pk_autotune": (I, [C.c_char_p, LL, LL, LL, C.c_char_p, C.c_char_p]),
    "pk_synth_normal_bf16": (None, [U64, U64, D, D, P, I64]),
    "pk_synth_normal_f32": (None, [U64, U64, D, D, P, I64]),
    "pk_synth_mask_bf16": (None, [U64, U64, D, P, I64]),
}

_lib = None


def load() -> C.CDLL:
    """Load the in-tree library (built by polykernel_amd.build / __graft_entry__.build)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m polykernel_amd.build` "
            "(the kernels have no CPU fallback)"
        )
    lib = C.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    msg = load().pk_last_error()
    return msg.decode() if msg else ""


def check(rc: int, name: str) -> None:
    if rc != PK_OK:
        raise PolyKernelError(name, rc, last_error())


def last_text() -> str:
    """Text result of the last runtime call that produced one (pk_last_text)."""
    t = load().pk_last_text()
    return t.decode() if t else ""
