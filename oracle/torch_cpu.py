"""PyTorch-CPU restatement of the reference's CPU path (test infrastructure / CPU baseline only).

The reference's "reference CPU path" is plain torch code run on the host (kernels/reference.py:
9-45, with unpack_int4 from kernels/quant.py:31-35 and dequantize_fp8 from kernels/fp8.py:33-35).
This module restates those steps with torch ops on CPU tensors, so that `bench.py`'s
`cpu_baseline` leg times the same op sequence on all host cores (torch's intra-op thread pool)
rather than a numpy port. It is pinned against the numpy oracle (`oracle.reference`,
`oracle.fp8`) in tests/test_oracle_torch_cpu.py: dequantized weights and the RMSNorm residual bit
for bit, RMSNorm and SwiGLU outputs within one fp16 step (reduction order, exp), the fp32 matmuls
within fp32 reduction-order tolerance of a float64 product.

The product package (`kernels.*`) never imports it.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def unpack_int4(qweight: torch.Tensor) -> torch.Tensor:
    """int32 [K/8, N] -> int32 [K, N] in 0..15: nibble i of packed row r is row 8r + i."""
    R, N = qweight.shape
    nibbles = [(qweight >> (4 * i)) & 0xF for i in range(8)]  # arithmetic shift, then mask
    return torch.stack(nibbles, dim=1).reshape(R * 8, N)


def dequantize_ref(qweight, scales, zeros, group_size: int = 128) -> torch.Tensor:
    """[N, K] in the scales' dtype: (q - z) * s with one rounding (reference.py:27-36)."""
    q = unpack_int4(qweight)
    K = q.shape[0]
    s = torch.repeat_interleave(scales, group_size, dim=0)[:K]
    z = torch.repeat_interleave(zeros, group_size, dim=0)[:K]
    return ((q.to(scales.dtype) - z) * s).t().contiguous()


def w4a16_ref(x, qweight, scales, zeros, group_size: int = 128, bias=None) -> torch.Tensor:
    """fp32 x @ dequant(W).T (+ bias), dequantizing on every call (reference.py:39-45)."""
    w = dequantize_ref(qweight, scales, zeros, group_size)
    y = torch.matmul(x.float(), w.float().t())
    return y if bias is None else y + bias.float()


def rmsnorm_ref(x, weight, eps: float = 1e-6, residual=None):
    """Optional fp16 residual add, fp32 mean of squares, fp16 normalized value times the weight
    (reference.py:9-19). Returns out, or (out, x + residual)."""
    h16 = x if residual is None else x + residual
    h = h16.float()
    normed = (h * torch.rsqrt(h.square().mean(dim=-1, keepdim=True) + eps)).to(h16.dtype)
    out = weight * normed
    return out if residual is None else (out, h16)


def swiglu_ref(gate, up) -> torch.Tensor:
    """F.silu(gate) * up in the inputs' dtype (reference.py:22-24)."""
    return F.silu(gate) * up


def dequantize_fp8(wq: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """e4m3 [K, N] and per-channel scale [N] -> [N, K] in the scale's dtype (fp8.py:33-35)."""
    return (scale.float().unsqueeze(1) * wq.float().t()).to(scale.dtype)


def w8a16_ref(x, wq, scale, bias=None) -> torch.Tensor:
    """fp32 x @ dequantize_fp8(wq, scale).T (+ bias), the reference's test reference
    (tests/test_fp8.py:20)."""
    y = torch.matmul(x.float(), dequantize_fp8(wq, scale).float().t())
    return y if bias is None else y + bias.float()
