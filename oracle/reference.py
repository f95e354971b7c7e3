"""Numpy restatement of the reference's PyTorch references (test infrastructure only).

Restates `kernels/reference.py:9-45` of the reference with the same rounding steps:

- fp16 arithmetic on fp16 operands is evaluated as one IEEE round-to-nearest-even of the exact
  result (numpy float16 ufuncs compute in float32 and round once; for a single add or multiply of
  two fp16 values this equals the exactly rounded result, which is also what torch does).
- float32 reductions follow numpy's pairwise order; callers compare reductions with tolerances.
"""

from __future__ import annotations

import numpy as np

from oracle.quant import unpack_int4


def dequantize_ref(qweight, scales, zeros, group_size: int = 128) -> np.ndarray:
    """[K/8, N] int4 -> [N, K] in scales' dtype; one rounding of (q - z) * s (reference.py:27-36).

    `q - z` is an exact small integer, so for fp16 scales this is exactly RNE((q - z) * s)."""
    q = unpack_int4(qweight)
    K, N = q.shape
    scales = np.asarray(scales)
    zeros = np.asarray(zeros)
    s = np.repeat(scales, group_size, axis=0)[:K]
    z = np.repeat(zeros, group_size, axis=0)[:K]
    w = (q.astype(scales.dtype) - z) * s
    return np.ascontiguousarray(w.T)


def w4a16_ref(x, qweight, scales, zeros, group_size: int = 128, bias=None) -> np.ndarray:
    """float32 x @ dequant(W).T (+ bias), reference.py:39-45. Returns float32 [M, N]."""
    w = dequantize_ref(qweight, scales, zeros, group_size)
    out = np.asarray(x, dtype=np.float32) @ w.astype(np.float32).T
    if bias is not None:
        out = out + np.asarray(bias).astype(np.float32)
    return out


def w4a16_ref_f64(x, qweight, scales, zeros, group_size: int = 128, bias=None) -> np.ndarray:
    """Same as `w4a16_ref` with float64 accumulation (a tighter target for tolerance checks)."""
    w = dequantize_ref(qweight, scales, zeros, group_size)
    out = np.asarray(x, dtype=np.float64) @ w.astype(np.float64).T
    if bias is not None:
        out = out + np.asarray(bias).astype(np.float64)
    return out


def rmsnorm_ref(x, weight, eps: float = 1e-6, residual=None):
    """Qwen2 RMSNorm with the optional fused residual add (reference.py:9-19).

    x, residual, weight: fp16. Returns `out` or `(out, x + residual)`."""
    x = np.asarray(x)
    if residual is not None:
        x = x + np.asarray(residual)  # fp16 add, one rounding
    h = x.astype(np.float32)
    var = np.mean(h * h, axis=-1, keepdims=True, dtype=np.float32)
    r = np.float32(1.0) / np.sqrt(var + np.float32(eps))  # torch.rsqrt on CPU: 1 / sqrt
    normed = (h * r).astype(x.dtype)
    out = np.asarray(weight) * normed  # fp16 multiply, one rounding
    return out if residual is None else (out, x)


def rmsnorm_parts(x, weight, eps: float = 1e-6, residual=None):
    """rmsnorm_ref with its fp16 intermediate exposed: returns (h, normed, out), where h is the
    (residual-added) fp16 input, normed = fp16(h * rsqrt(mean(h^2) + eps)) and out = w * normed."""
    x = np.asarray(x)
    h = x if residual is None else x + np.asarray(residual)
    hf = h.astype(np.float32)
    var = np.mean(hf * hf, axis=-1, keepdims=True, dtype=np.float32)
    normed = (hf * (np.float32(1.0) / np.sqrt(var + np.float32(eps)))).astype(h.dtype)
    return h, normed, np.asarray(weight) * normed


def silu_ref(gate) -> np.ndarray:
    """F.silu on fp16: g / (1 + exp(-g)) in float32, rounded once to the input dtype."""
    g = np.asarray(gate)
    g32 = g.astype(np.float32)
    with np.errstate(over="ignore"):
        s = g32 / (np.float32(1.0) + np.exp(-g32))
    return s.astype(g.dtype)


def swiglu_ref(gate, up) -> np.ndarray:
    """silu(gate) * up in fp16 (reference.py:22-24)."""
    return silu_ref(gate) * np.asarray(up)


def rmsnorm_bytes(M: int, N: int, residual: bool, elem: int = 2) -> int:
    """Minimum traffic of fused RMSNorm(+residual) (kernels/rmsnorm.py:71-74)."""
    return (4 if residual else 2) * M * N * elem + N * elem


def swiglu_bytes(M: int, I: int, elem: int = 2) -> int:
    """Minimum traffic of SwiGLU: read gate and up, write out (kernels/swiglu.py:64-65)."""
    return 3 * M * I * elem
