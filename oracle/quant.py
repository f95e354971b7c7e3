"""int4 weight format and RTN quantizer (numpy restatement; test infrastructure only).

Restates `kernels/quant.py` of the reference:

- layout (`quant.py:3-10`): for a linear weight W [N, K], `qweight` is int32 [K/8, N]; nibble i
  (bits 4i..4i+3) of word [r, n] holds q[8r+i, n] in 0..15. `scales` and `zeros` are
  [K/group, N] in the weight's dtype (fp16 for an fp16 weight). Dequantized value:
  (q - zero) * scale.
- RTN (`quant.py:38-49`): per group of `group_size` consecutive K, in float32,
  scale = max((wmax - wmin) / 15, 1e-6), zero = clamp(round(-wmin / scale), 0, 15),
  q = clamp(round(w / scale + zero), 0, 15); round is half-to-even (`torch.round`).
"""

from __future__ import annotations

import numpy as np

PACK = 8  # int4 values per int32 (quant.py:17)


def pack_int4(q: np.ndarray) -> np.ndarray:
    """[K, N] integers in 0..15 -> [K/8, N] int32 (quant.py:20-28)."""
    q = np.asarray(q)
    K, N = q.shape
    assert K % PACK == 0, "K must be a multiple of 8"
    q64 = q.astype(np.uint64).reshape(K // PACK, PACK, N)
    shifts = (np.arange(PACK, dtype=np.uint64) * np.uint64(4)).reshape(1, PACK, 1)
    packed = (q64 << shifts).sum(axis=1, dtype=np.uint64)  # < 2**32
    # Two's-complement reinterpretation to int32, as quant.py:27 does with `packed - 2**32`.
    return packed.astype(np.uint32).view(np.int32)


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """[K/8, N] int32 -> [K, N] int32 in 0..15 (quant.py:31-35): arithmetic >> then & 0xF."""
    packed = np.asarray(packed, dtype=np.int32)
    shifts = (np.arange(PACK, dtype=np.int32) * 4).reshape(1, PACK, 1)
    q = (packed[:, None, :] >> shifts) & 0xF
    return q.reshape(-1, packed.shape[1]).astype(np.int32)


def quantize_rtn(weight: np.ndarray, group_size: int = 128):
    """RTN asymmetric int4 quantization of an [N, K] weight (quant.py:38-49).

    Returns (qweight int32 [K/8, N], scale [K/G, N], zero [K/G, N]); scale and zero are cast to
    the weight's dtype (float16 for a float16 weight, float32 for float32), as `quant.py:49`.
    """
    weight = np.asarray(weight)
    N, K = weight.shape
    assert K % group_size == 0, f"K={K} must be a multiple of group_size={group_size}"
    w = weight.T.astype(np.float32).reshape(K // group_size, group_size, N)
    wmin = w.min(axis=1)
    wmax = w.max(axis=1)
    scale = np.maximum((wmax - wmin) / np.float32(15), np.float32(1e-6)).astype(np.float32)
    zero = np.clip(np.rint(-wmin / scale), 0, 15).astype(np.float32)
    q = np.clip(np.rint(w / scale[:, None, :] + zero[:, None, :]), 0, 15)
    qweight = pack_int4(q.reshape(K, N).astype(np.int32))
    return qweight, scale.astype(weight.dtype), zero.astype(weight.dtype)


def weight_bytes(N: int, K: int, group_size: int = 128) -> int:
    """Packed int4 plus fp16 scales and zeros (quant.py:52-54)."""
    return N * K // 2 + 2 * (K // group_size) * N * 2
