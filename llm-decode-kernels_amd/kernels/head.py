"""Tied fp16 lm_head at one decode row on the GPU (libldk_amd.so `ldk_f16_gemv`).

`lm_head(h, weight)` computes `F.linear(h, weight)` for a single fp16 row h [..., K] against the
fp16 table weight [N, K]: the last step of the reference's runner forward
(kernels/e2e/model.py:253) on the fp16-head backends. One launch streams the table once with
non-temporal 16-byte loads (fp32 accumulation, fp16 output). It is used only where it applies
(one row, fp16, K a multiple of 8 up to 2048, 16-byte aligned operands); `applies` says so, and
callers use the library GEMM otherwise.
"""

from __future__ import annotations

import torch

from kernels import _lib


def applies(h: torch.Tensor, weight: torch.Tensor) -> bool:
    """True when `lm_head` takes this (h, weight) pair."""
    K = h.shape[-1]
    return (h.is_cuda and weight.is_cuda and h.dtype == torch.float16 and weight.dtype == torch.float16
            and h.numel() == K and weight.dim() == 2 and weight.shape[1] == K and weight.stride(1) == 1
            and K % 8 == 0 and K <= 2048 and weight.stride(0) % 8 == 0
            and weight.data_ptr() % 16 == 0)


def _row(t: torch.Tensor, K: int, name: str) -> torch.Tensor:
    if t.numel() != K or t.dtype != torch.float16:
        raise ValueError(f"lm_head: {name} must be one fp16 row of {K}, got {tuple(t.shape)} {t.dtype}")
    r = t.reshape(K)
    return r if r.stride(0) == 1 and r.data_ptr() % 16 == 0 else r.contiguous()


def lm_head(h: torch.Tensor, weight: torch.Tensor, rows_per_wave: int = 0,
            norm_weight: torch.Tensor | None = None, eps: float = 1e-6,
            residual: torch.Tensor | None = None) -> torch.Tensor:
    """h: fp16 [..., K] holding one row; weight: fp16 [N, K] (row stride a multiple of 8).
    Returns fp16 [..., N] like F.linear(h, weight). With norm_weight, the row is first
    `rmsnorm(h, norm_weight, eps, residual)` (kernels/reference.py:9-19) inside the same launch:
    the final norm and the head of the runner (kernels/e2e/model.py:250-253)."""
    K = h.shape[-1]
    if h.numel() != K:
        raise ValueError(f"lm_head: one row expected, got shape {tuple(h.shape)}")
    if weight.dim() != 2 or weight.shape[1] != K or weight.stride(1) != 1:
        raise ValueError(f"lm_head: weight must be [N, {K}] with unit column stride, got "
                         f"{tuple(weight.shape)} strides {weight.stride()}")
    if h.dtype != torch.float16 or weight.dtype != torch.float16:
        raise ValueError(f"lm_head: fp16 operands expected, got {h.dtype} and {weight.dtype}")
    x = _row(h, K, "h")
    nw = None if norm_weight is None else _row(norm_weight, K, "norm_weight")
    res = None if residual is None else _row(residual, K, "residual")
    if res is not None and nw is None:
        raise ValueError("lm_head: a residual needs norm_weight")
    dev = _lib.require_gpu(x, weight, nw, res, what="lm_head")
    N = weight.shape[0]
    y = torch.empty(*h.shape[:-1], N, dtype=torch.float16, device=dev)
    with _lib.device_guard(dev):
        if nw is None:
            st = _lib.load().ldk_f16_gemv(_lib.ptr(x), _lib.ptr(weight), weight.stride(0), _lib.ptr(y),
                                          N, K, rows_per_wave, _lib.stream(dev))
        else:
            st = _lib.load().ldk_f16_rmsnorm_gemv(_lib.ptr(x), _lib.ptr(res), _lib.ptr(nw), float(eps),
                                                  _lib.ptr(weight), weight.stride(0), _lib.ptr(y), N, K,
                                                  rows_per_wave, _lib.stream(dev))
    _lib.check(st, "lm_head")
    return y
