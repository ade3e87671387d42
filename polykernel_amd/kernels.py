"""Torch-tensor front end of the gfx950 kernels.

Function names and argument meaning follow the reference's golden interface
(tests/golden/golden.py:48-172, tests/golden/quant_golden.py:71-101): bf16 in,
bf16 out, fused ops equal to their compositions.  Tensors are device tensors
(torch is only the allocator and stream provider); every call goes through the
C-ABI of libpolykernel_amd.so on torch's current stream.  A failing launch
raises PolyKernelError with the library's message.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import check

bf16 = torch.bfloat16


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _dev(t: torch.Tensor, dtype: torch.dtype, name: str) -> int:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name}: expected a torch.Tensor")
    if not t.is_cuda:
        raise ValueError(f"{name}: tensor must live on a GPU (got {t.device})")
    if t.dtype != dtype:
        raise TypeError(f"{name}: expected {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name}: tensor must be contiguous")
    return t.data_ptr()


def _opt(t: Optional[torch.Tensor], dtype, name) -> Optional[int]:
    return None if t is None else _dev(t, dtype, name)


def rmsnorm(x: torch.Tensor, weight: Optional[torch.Tensor] = None, eps: float = 1e-5) -> torch.Tensor:
    """golden.rmsnorm (golden.py:83-90) via launch_rmsnorm."""
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    out = torch.empty_like(x)
    check(_lib.load().launch_rmsnorm(_dev(x, bf16, "x"), _opt(weight, bf16, "weight"),
                                     _dev(out, bf16, "out"), rows, cols, eps, _stream()),
          "launch_rmsnorm")
    return out


def fused_residual_rmsnorm(x: torch.Tensor, residual: torch.Tensor,
                           weight: Optional[torch.Tensor] = None, eps: float = 1e-5,
                           config: Optional[dict] = None) -> torch.Tensor:
    """golden.fused_residual_rmsnorm (golden.py:108-112); `config` picks one of
    pk_op_configs("fused_residual_rmsnorm", rows, cols, 0) (tuning/test hook
    pk_fused_residual_rmsnorm_config)."""
    if x.shape != residual.shape:
        raise ValueError("x and residual must have the same shape")
    cols = x.shape[-1]
    rows = x.numel() // cols
    out = torch.empty_like(x)
    args = (_dev(x, bf16, "x"), _dev(residual, bf16, "residual"), _opt(weight, bf16, "weight"),
            _dev(out, bf16, "out"), rows, cols, eps)
    if config is None:
        check(_lib.load().launch_fused_residual_rmsnorm(*args, _stream()), "launch_fused_residual_rmsnorm")
    else:
        check(_lib.load().pk_fused_residual_rmsnorm_config(*args, _lib.Config(**config), _stream()),
              "pk_fused_residual_rmsnorm_config")
    return out


def gelu(x: torch.Tensor) -> torch.Tensor:
    """golden.gelu (golden.py:63-66); bit-exact with kernels/cpu launch_gelu_cpu."""
    out = torch.empty_like(x)
    check(_lib.load().launch_gelu(_dev(x, bf16, "x"), _dev(out, bf16, "out"), x.numel(), _stream()),
          "launch_gelu")
    return out


def softmax(x: torch.Tensor) -> torch.Tensor:
    """golden.softmax over the last axis (golden.py:75-80)."""
    cols = x.shape[-1]
    out = torch.empty_like(x)
    check(_lib.load().launch_softmax(_dev(x, bf16, "x"), _dev(out, bf16, "out"),
                                     x.numel() // cols, cols, _stream()), "launch_softmax")
    return out


def fused_softmax_mask(logits: torch.Tensor, mask: torch.Tensor, config: Optional[dict] = None) -> torch.Tensor:
    """golden.fused_softmax_mask (golden.py:115-117) on fp32 logits + bf16 additive mask;
    `config` picks one of pk_op_configs("fused_softmax_mask", rows, cols, 0)
    (tuning/test hook pk_fused_softmax_mask_config)."""
    if logits.shape != mask.shape:
        raise ValueError("logits and mask must have the same shape")
    cols = logits.shape[-1]
    out = torch.empty(logits.shape, dtype=bf16, device=logits.device)
    args = (_dev(logits, torch.float32, "logits"), _dev(mask, bf16, "mask"), _dev(out, bf16, "out"),
            logits.numel() // cols, cols)
    if config is None:
        check(_lib.load().launch_fused_softmax_mask(*args, _stream()), "launch_fused_softmax_mask")
    else:
        check(_lib.load().pk_fused_softmax_mask_config(*args, _lib.Config(**config), _stream()),
              "pk_fused_softmax_mask_config")
    return out


def _mk(a: torch.Tensor, b: torch.Tensor) -> Tuple[int, int, int]:
    K = a.shape[-1]
    if b.dim() != 2 or b.shape[0] != K:
        raise ValueError(f"contraction mismatch: a[..., {K}] @ b{tuple(b.shape)}")
    return a.numel() // K, b.shape[1], K


def matmul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """golden.matmul (golden.py:58-60): [..., M, K] @ [K, N]."""
    M, N, K = _mk(a, b)
    out = torch.empty(*a.shape[:-1], N, dtype=bf16, device=a.device)
    check(_lib.load().launch_matmul(_dev(a, bf16, "a"), _dev(b, bf16, "b"), _dev(out, bf16, "out"),
                                    M, N, K, _stream()), "launch_matmul")
    return out


def gemm_ex(epi: int, a, b, bias=None, residual=None, tile: int = -1) -> torch.Tensor:
    """Explicit-tile GEMM (tuning/test hook pk_gemm_ex)."""
    M, N, K = _mk(a, b)
    out = torch.empty(*a.shape[:-1], N, dtype=bf16, device=a.device)
    check(_lib.load().pk_gemm_ex(epi, _dev(a, bf16, "a"), _dev(b, bf16, "b"), _dev(out, bf16, "out"),
                                 _opt(bias, bf16, "bias"), _opt(residual, bf16, "residual"),
                                 M, N, K, tile, _stream()), "pk_gemm_ex")
    return out


def fused_rmsnorm_matmul(x: torch.Tensor, w: torch.Tensor, weight: Optional[torch.Tensor] = None,
                         eps: float = 1e-5) -> torch.Tensor:
    """golden.fused_rmsnorm_matmul (golden.py:96-100); `weight` is the rmsnorm gamma."""
    M, N, K = _mk(x, w)
    out = torch.empty(*x.shape[:-1], N, dtype=bf16, device=x.device)
    lib = _lib.load()
    if weight is None:
        rc = lib.launch_fused_rmsnorm_matmul(_dev(x, bf16, "x"), _dev(w, bf16, "w"),
                                             _dev(out, bf16, "out"), M, N, K, eps, _stream())
        check(rc, "launch_fused_rmsnorm_matmul")
    else:
        rc = lib.launch_fused_rmsnorm_matmul_gamma(_dev(x, bf16, "x"), _dev(weight, bf16, "weight"),
                                                   _dev(w, bf16, "w"), _dev(out, bf16, "out"),
                                                   M, N, K, eps, _stream())
        check(rc, "launch_fused_rmsnorm_matmul_gamma")
    return out


def fused_matmul_bias_gelu(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """golden.fused_matmul_bias_gelu (golden.py:103-105)."""
    M, N, K = _mk(x, w)
    out = torch.empty(*x.shape[:-1], N, dtype=bf16, device=x.device)
    check(_lib.load().launch_fused_matmul_bias_gelu(_dev(x, bf16, "x"), _dev(w, bf16, "w"),
                                                    _dev(b, bf16, "b"), _dev(out, bf16, "out"),
                                                    M, N, K, _stream()),
          "launch_fused_matmul_bias_gelu")
    return out


def fused_matmul_bias_residual(x: torch.Tensor, w: torch.Tensor, b: Optional[torch.Tensor],
                               residual: torch.Tensor) -> torch.Tensor:
    """add(bias(matmul(x, w), b), residual) -- the MLP down-projection epilogue."""
    M, N, K = _mk(x, w)
    out = torch.empty(*x.shape[:-1], N, dtype=bf16, device=x.device)
    check(_lib.load().launch_fused_matmul_bias_residual(
        _dev(x, bf16, "x"), _dev(w, bf16, "w"), _opt(b, bf16, "b"), _dev(residual, bf16, "residual"),
        _dev(out, bf16, "out"), M, N, K, _stream()), "launch_fused_matmul_bias_residual")
    return out


def mlp_block(x, gamma, w1, b1, w2, b2, eps: float = 1e-6, workspace: Optional[torch.Tensor] = None):
    """RMSNorm -> MatMul W1 + b1 -> GELU -> MatMul W2 + b2 -> + x (config-2 block)."""
    M, d = x.numel() // x.shape[-1], x.shape[-1]
    F = w1.shape[1]
    lib = _lib.load()
    need = lib.pk_mlp_block_workspace_size(M, d, F)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    out = torch.empty_like(x)
    check(lib.launch_mlp_block(_dev(x, bf16, "x"), _opt(gamma, bf16, "gamma"), _dev(w1, bf16, "w1"),
                               _dev(b1, bf16, "b1"), _dev(w2, bf16, "w2"), _dev(b2, bf16, "b2"),
                               _dev(out, bf16, "out"), M, d, F, eps, workspace.data_ptr(),
                               workspace.numel(), _stream()), "launch_mlp_block")
    return out


def kv_cache_update(cache: torch.Tensor, new: torch.Tensor) -> torch.Tensor:
    """Out-of-place KV append: concat(cache, new) on axis 2 (attention.cpp:63-92)."""
    B, H, Sc, D = cache.shape
    Sn = new.shape[2]
    out = torch.empty(B, H, Sc + Sn, D, dtype=bf16, device=cache.device)
    check(_lib.load().launch_kv_cache_update(_dev(cache, bf16, "cache"), _dev(new, bf16, "new"),
                                             _dev(out, bf16, "out"), B, H, Sc, Sn, D, _stream()),
          "launch_kv_cache_update")
    return out


def attention_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                      scale: Optional[float] = None, causal: bool = True) -> torch.Tensor:
    """SDPA over the full key set (attention.cpp:95-163)."""
    B, H, Sq, D = q.shape
    Skv = k.shape[2]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = torch.empty_like(q)
    check(_lib.load().launch_attention_prefill(_dev(q, bf16, "q"), _dev(k, bf16, "k"), _dev(v, bf16, "v"),
                                               _dev(out, bf16, "out"), B, H, Sq, Skv, D, scale,
                                               int(causal), _stream()), "launch_attention_prefill")
    return out


def fused_kv_append_attention(q, k_new, v_new, k_cache, v_cache, s_cache: int,
                              scale: Optional[float] = None, causal: bool = True) -> torch.Tensor:
    """In-place append of k_new/v_new at row s_cache of the caches, then attention
    over the s_cache + S_q keys (golden.fused_kv_append_attention, golden.py:139-172)."""
    B, H, Sq, D = q.shape
    cap = k_cache.shape[2]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    out = torch.empty_like(q)
    check(_lib.load().launch_fused_kv_append_attention(
        _dev(q, bf16, "q"), _dev(k_cache, bf16, "k_cache"), _dev(v_cache, bf16, "v_cache"),
        _dev(k_new, bf16, "k_new"), _dev(v_new, bf16, "v_new"), _dev(out, bf16, "out"),
        B, H, Sq, s_cache, D, cap, scale, int(causal), _stream()), "launch_fused_kv_append_attention")
    return out


def quantize_per_channel(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """quant_golden.quantize_per_channel (quant_golden.py:71-83), bit-exact."""
    K, N = w.shape
    wq = torch.empty(K, N, dtype=torch.int8, device=w.device)
    scale = torch.empty(N, dtype=torch.float32, device=w.device)
    check(_lib.load().launch_quantize_int8_per_channel(_dev(w, bf16, "w"), _dev(wq, torch.int8, "wq"),
                                                       _dev(scale, torch.float32, "scale"), K, N,
                                                       _stream()), "launch_quantize_int8_per_channel")
    return wq, scale


def matmul_int8(a: torch.Tensor, wq: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """quant_golden.matmul_int8 (quant_golden.py:91-101)."""
    K = a.shape[-1]
    M, N = a.numel() // K, wq.shape[1]
    out = torch.empty(*a.shape[:-1], N, dtype=bf16, device=a.device)
    check(_lib.load().launch_matmul_int8(_dev(a, bf16, "a"), _dev(wq, torch.int8, "wq"),
                                         _dev(scale, torch.float32, "scale"), _dev(out, bf16, "out"),
                                         M, N, K, _stream()), "launch_matmul_int8")
    return out


def int8_default_config(M: int, N: int, K: int) -> Optional[dict]:
    """Configuration launch_matmul_int8 picks for a shape (None: generic kernel)."""
    cfg = _lib.Config()
    rc = _lib.load().pk_int8_default_config(M, N, K, cfg)
    if rc == _lib.PK_ERR_UNSUPPORTED:
        return None
    check(rc, "pk_int8_default_config")
    return cfg.as_dict()


def matmul_int8_ex(epi: int, a: torch.Tensor, wq: torch.Tensor, scale: torch.Tensor,
                   residual: Optional[torch.Tensor] = None, config: Optional[dict] = None) -> torch.Tensor:
    """int8 matmul with an explicit epilogue (0 none, 1 GELU, 2 + residual) and
    launch configuration (tuning/test hook pk_matmul_int8_ex)."""
    K = a.shape[-1]
    M, N = a.numel() // K, wq.shape[1]
    out = torch.empty(*a.shape[:-1], N, dtype=bf16, device=a.device)
    cfg = None if config is None else _lib.Config(**config)
    check(_lib.load().pk_matmul_int8_ex(epi, _dev(a, bf16, "a"), _dev(wq, torch.int8, "wq"),
                                        _dev(scale, torch.float32, "scale"), _dev(out, bf16, "out"),
                                        _opt(residual, bf16, "residual"), M, N, K, cfg, None, 0,
                                        _stream()), "pk_matmul_int8_ex")
    return out


def decode_mlp_int8(x, w1q, s1, w2q, s2, workspace: Optional[torch.Tensor] = None):
    """add(matmul_int8(gelu(matmul_int8(x, W1q, s1)), W2q, s2), x) (config-5 chain)."""
    d = x.shape[-1]
    M = x.numel() // d
    F = w1q.shape[1]
    lib = _lib.load()
    need = lib.pk_decode_mlp_int8_workspace_size(M, d, F)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    out = torch.empty_like(x)
    check(lib.launch_decode_mlp_int8(_dev(x, bf16, "x"), _dev(w1q, torch.int8, "w1q"),
                                     _dev(s1, torch.float32, "s1"), _dev(w2q, torch.int8, "w2q"),
                                     _dev(s2, torch.float32, "s2"), _dev(out, bf16, "out"), M, d, F,
                                     workspace.data_ptr(), workspace.numel(), _stream()),
          "launch_decode_mlp_int8")
    return out
