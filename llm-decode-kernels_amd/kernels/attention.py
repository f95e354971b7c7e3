"""Fused decode attention on gfx950 (libldk_amd.so `ldk_decode_attention`): for one new token,
RoPE on q and k, the KV-cache write at `pos` and grouped-query softmax attention over positions
0..pos, one launch per layer.

It replaces, for decode steps, the attention block of the reference's Qwen2 runner
(kernels/e2e/model.py:212-243), which is about twenty small torch launches per layer.
"""

from __future__ import annotations

import torch

from kernels import _lib

MAX_LEN = 1 << 20
HEAD_DIM = 128


def supported(head_dim: int, max_len: int, batch: int, tokens: int) -> bool:
    """The kernel's domain: head_dim 128, one token of one sequence, and a cache length that is a
    multiple of 8 (its K^T rows are read 8 positions per 16-byte load)."""
    return (head_dim == HEAD_DIM and 8 <= max_len <= MAX_LEN and max_len % 8 == 0 and batch == 1
            and tokens == 1)


def decode_attention(qkv: torch.Tensor, pos: torch.Tensor, inv_freq: torch.Tensor,
                     kt_cache: torch.Tensor, v_cache: torch.Tensor, n_heads: int, n_kv: int,
                     scale: float) -> torch.Tensor:
    """qkv [..., (n_heads + 2 n_kv) * 128] fp16 (one token); pos int64 [1]; inv_freq fp32 [64];
    kt_cache [1, n_kv, 128, L] and v_cache [1, n_kv, L, 128] fp16 of this layer (updated at
    pos). Returns the attention output [1, 1, n_heads * 128] fp16."""
    hd = HEAD_DIM
    assert qkv.shape[-1] == (n_heads + 2 * n_kv) * hd and qkv.numel() == qkv.shape[-1]
    assert kt_cache.shape[-3:-1] == (n_kv, hd) and v_cache.shape[-3] == n_kv
    assert kt_cache.is_contiguous() and v_cache.is_contiguous()
    L = kt_cache.shape[-1]
    if qkv.dtype != torch.float16 or kt_cache.dtype != torch.float16:
        raise ValueError("decode_attention: qkv and the cache must be float16")
    if pos.dtype != torch.int64 or inv_freq.dtype != torch.float32:
        raise ValueError("decode_attention: pos int64, inv_freq float32")
    q = qkv.reshape(-1)
    if q.stride(0) != 1:
        q = q.contiguous()
    dev = _lib.require_gpu(q, pos, inv_freq, kt_cache, v_cache, what="decode_attention")
    out = torch.empty((1, 1, n_heads * hd), dtype=torch.float16, device=dev)
    with _lib.device_guard(dev):
        st = _lib.load().ldk_decode_attention(
            _lib.ptr(q), _lib.ptr(pos), _lib.ptr(inv_freq.contiguous()), _lib.ptr(kt_cache),
            _lib.ptr(v_cache), _lib.ptr(out), n_heads, n_kv, hd, L, float(scale), _lib.stream(dev))
    _lib.check(st, "decode_attention")
    return out
