"""OCP FP8 e4m3 (float8_e4m3fn) weights: numpy restatement (test infrastructure only).

Restates `kernels/fp8.py:21-39` and the W8A16 reference of `tests/test_fp8.py:20`:

- `quantize_fp8` (fp8.py:25-30): per output channel n, scale = max(absmax_k |w| / 448, 1e-12) in
  float32; wq = e4m3(clamp(w / scale, -448, 448)) with round-to-nearest-even, stored [K, N];
  scale is returned in the weight's dtype (the division uses the float32 scale).
- `dequantize_fp8` (fp8.py:33-35): (wq.float() * scale.float()).to(scale.dtype), [N, K].
- e4m3fn (OCP): 1 sign, 4 exponent (bias 7), 3 mantissa bits; no infinities; 0x7F/0xFF are NaN;
  largest finite 448; subnormals m * 2^-9.

The encoder is written from the format's definition (nearest representable value, ties to the
even code), not from any library's conversion routine; tests pin it against torch's
`float8_e4m3fn` cast, the routine the reference calls at fp8.py:29.
"""

from __future__ import annotations

import numpy as np

FP8_MAX = 448.0


def _positive_table() -> np.ndarray:
    """Values of the finite non-negative codes 0x00..0x7E, ascending (the code order)."""
    vals = np.empty(127, dtype=np.float64)
    for c in range(127):
        e, m = c >> 3, c & 7
        vals[c] = m * 2.0**-9 if e == 0 else 2.0 ** (e - 7) * (1 + m / 8)
    return vals


_POS = _positive_table()


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """uint8 e4m3fn codes -> float32 (NaN for 0x7F/0xFF)."""
    codes = np.asarray(codes, dtype=np.uint8)
    mag = codes & 0x7F
    out = np.where(mag == 0x7F, np.nan, _POS[np.minimum(mag, 126)])
    out = np.where(codes & 0x80, -out, out)
    return out.astype(np.float32)


def e4m3_encode(v: np.ndarray) -> np.ndarray:
    """float32 values with |v| <= 448 -> uint8 e4m3fn codes, round to nearest, ties to even.

    The sign of zero is kept (-0.0 -> 0x80), as a sign-magnitude conversion does."""
    v = np.asarray(v, dtype=np.float32)
    a = np.abs(v).astype(np.float64)
    assert np.all(a <= FP8_MAX), "e4m3_encode expects values already clamped to +-448"
    hi = np.searchsorted(_POS, a, side="left")  # _POS[hi-1] < a <= _POS[hi]
    hi = np.minimum(hi, 126)
    lo = np.maximum(hi - 1, 0)
    d_lo = a - _POS[lo]
    d_hi = _POS[hi] - a
    exact = d_hi == 0
    pick_hi = exact | (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    sign = np.signbit(v)
    return np.where(sign, code | 0x80, code).astype(np.uint8)


def quantize_fp8(weight: np.ndarray):
    """[N, K] weight -> (wq uint8 e4m3 codes [K, N], scale [N] in weight's dtype), fp8.py:25-30."""
    weight = np.asarray(weight)
    w = weight.astype(np.float32)
    scale = np.maximum(np.abs(w).max(axis=1) / np.float32(FP8_MAX), np.float32(1e-12))
    scale = scale.astype(np.float32)
    wq = e4m3_encode(np.clip(w / scale[:, None], -FP8_MAX, FP8_MAX).astype(np.float32))
    return np.ascontiguousarray(wq.T), scale.astype(weight.dtype)


def dequantize_fp8(wq: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """wq codes [K, N], scale [N] -> [N, K] in scale's dtype (fp8.py:33-35)."""
    scale = np.asarray(scale)
    w = e4m3_decode(wq).T.astype(np.float32) * scale.astype(np.float32)[:, None]
    return np.ascontiguousarray(w.astype(scale.dtype))


def w8a16_ref(x, wq, scale, bias=None) -> np.ndarray:
    """float32 x @ dequant(W).T (+ bias), as tests/test_fp8.py:20. Returns float32 [M, N]."""
    out = np.asarray(x, dtype=np.float32) @ dequantize_fp8(wq, scale).astype(np.float32).T
    if bias is not None:
        out = out + np.asarray(bias).astype(np.float32)
    return out


def fp8_bytes(N: int, K: int) -> int:
    """fp8 weight plus fp16 per-channel scale (fp8.py:38-39)."""
    return N * K + N * 2
