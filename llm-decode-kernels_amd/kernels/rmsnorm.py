"""Fused RMSNorm (+ residual add) on gfx950.

Drop-in for the reference's `kernels/rmsnorm.py`. One workgroup normalizes one row; with a
residual, the kernel also writes `x + residual` (the next block's residual stream), so every
element is read once and written once. Rounding steps follow the reference (Qwen2/HF numerics,
kernels/reference.py:9-19): fp16 residual add, fp32 mean of squares, fp16 normalized value, fp16
multiply by the weight.
"""

from __future__ import annotations

import torch

from kernels import _lib


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6, residual=None):
    """RMSNorm over the last dim. Returns `out`, or `(out, x + residual)` with a residual
    (rmsnorm.py:44-68)."""
    shape = x.shape
    N = shape[-1]
    x2 = x.reshape(-1, N)
    assert x2.stride(-1) == 1 and weight.is_contiguous()
    dev = _lib.require_gpu(x, weight, residual, what="rmsnorm")
    if x.dtype != torch.float16 or weight.dtype != torch.float16:
        raise ValueError("rmsnorm: x and weight must be float16")
    M = x2.shape[0]
    out = torch.empty((M, N), dtype=x.dtype, device=dev)
    r2 = res_out = None
    if residual is not None:
        r2 = residual.reshape(-1, N)
        if r2.stride(-1) != 1:
            r2 = r2.contiguous()
        res_out = torch.empty_like(out)
    with _lib.device_guard(dev):
        st = _lib.load().ldk_rmsnorm(
            _lib.ptr(x2), x2.stride(0), _lib.ptr(r2), 0 if r2 is None else r2.stride(0),
            _lib.ptr(weight), _lib.ptr(out), out.stride(0), _lib.ptr(res_out),
            0 if res_out is None else res_out.stride(0), M, N, float(eps), _lib.stream(dev))
    _lib.check(st, "rmsnorm")
    if residual is None:
        return out.view(shape)
    return out.view(shape), res_out.view(shape)


def rmsnorm_bytes(M: int, N: int, residual: bool, elem: int = 2) -> int:
    """Minimum DRAM traffic: read x (+ residual) and weight, write out (+ new residual)
    (rmsnorm.py:71-74)."""
    tensors = 4 if residual else 2
    return tensors * M * N * elem + N * elem
