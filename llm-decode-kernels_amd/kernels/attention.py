"""Fused attention on gfx950 (libldk_amd.so): `decode_attention` (`ldk_decode_attention`) for
one new token, RoPE on q and k, the KV-cache write at `pos` and grouped-query softmax attention
over positions 0..pos, one launch per layer; `prefill_attention` (`ldk_prefill_attention`) the
same for the T tokens of a prompt, causal, in two launches.

It replaces, for decode steps, the attention block of the reference's Qwen2 runner
(kernels/e2e/model.py:212-243), which is about twenty small torch launches per layer.
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from kernels import _lib

MAX_LEN = 1 << 20
HEAD_DIM = 128
CHUNK = 32  # positions per cache tile row set; max_len is a multiple of it

# The cache is kept in the matrix cores' operand order, in 1 KB tiles (each one 16-byte load per
# lane of a wave). For head_dim 128 (the kernel's; the torch helpers take any multiple of 32):
#  K, per kv head: [max_len/32 chunks][2 row halves hb][4 dim steps s][16 rows i][32 dims], row i
#    of half hb of chunk c holding position 32c + 8(i // 4) + 4hb + i % 4, dims 32s .. 32s + 31;
#  V^T, per kv head: [max_len/32 steps][8 dim blocks][16 dims][32 positions].


def k_cache_shape(n_kv: int, max_len: int, head_dim: int = HEAD_DIM) -> tuple:
    return (n_kv, max_len // CHUNK, 2, head_dim // 32, 16, 32)


def vt_cache_shape(n_kv: int, max_len: int, head_dim: int = HEAD_DIM) -> tuple:
    return (n_kv, max_len // CHUNK, head_dim // 16, 16, 32)


def k_to_tiles(k: torch.Tensor) -> torch.Tensor:
    """k [..., n_kv, L, hd] (the reference's layout) -> K tiles [..., n_kv, L/32, 2, hd/32, 16, 32]."""
    *lead, L, hd = k.shape
    assert hd % 32 == 0 and L % CHUNK == 0
    n = len(lead)
    # position 32c + 8a + 4hb + r, dim 32s + e  ->  tile (c, hb, s), row 4a + r, column e
    x = k.reshape(*lead, L // CHUNK, 4, 2, 4, hd // 32, 32)  # (c, a, hb, r, s, e)
    x = x.permute(*range(n), n, n + 2, n + 4, n + 1, n + 3, n + 5)  # (c, hb, s, a, r, e)
    return x.reshape(*lead, L // CHUNK, 2, hd // 32, 16, 32)


def k_from_tiles(t: torch.Tensor) -> torch.Tensor:
    """K tiles [..., n_kv, L/32, 2, hd/32, 16, 32] -> k [..., n_kv, L, hd]."""
    *lead, nc, _, ns, _, _ = t.shape
    n = len(lead)
    x = t.reshape(*lead, nc, 2, ns, 4, 4, 32)  # (c, hb, s, a, r, e)
    x = x.permute(*range(n), n, n + 3, n + 1, n + 4, n + 2, n + 5)  # (c, a, hb, r, s, e)
    return x.reshape(*lead, nc * CHUNK, ns * 32)


def vt_to_tiles(v: torch.Tensor) -> torch.Tensor:
    """v [..., n_kv, L, hd] (the reference's layout) -> V^T tiles [..., n_kv, L/32, hd/16, 16, 32]."""
    *lead, L, hd = v.shape
    assert hd % 16 == 0 and L % CHUNK == 0
    n = len(lead)
    x = v.reshape(*lead, L // CHUNK, 32, hd // 16, 16)  # (t, p, b, e)
    return x.permute(*range(n), n, n + 2, n + 3, n + 1).contiguous()  # (t, b, e, p)


def v_from_tiles(t: torch.Tensor) -> torch.Tensor:
    """V^T tiles [..., n_kv, L/32, hd/16, 16, 32] -> v [..., n_kv, L, hd]."""
    *lead, nt, nb, _, _ = t.shape
    n = len(lead)
    x = t.permute(*range(n), n, n + 3, n + 1, n + 2)  # (t, p, b, e)
    return x.reshape(*lead, nt * CHUNK, nb * 16)


def write_kv(k_tiles: torch.Tensor, vt_tiles: torch.Tensor, pos: torch.Tensor, k: torch.Tensor,
             v: torch.Tensor) -> None:
    """Write k, v [B, n_kv, T, hd] at positions pos [T] (int64) into one layer's tiled caches
    k_tiles [B, n_kv, L/32, 2, hd/32, 16, 32] and vt_tiles [B, n_kv, L/32, hd/16, 16, 32]."""
    B, nkv, T, hd = k.shape
    c, q = pos // CHUNK, pos % CHUNK
    hb, i = (q // 4) % 2, 4 * (q // 8) + q % 4
    # advanced indices split by slices put the position dimension first: [T, B, n_kv, ...]
    k_tiles[:, :, c, hb, :, i, :] = k.reshape(B, nkv, T, hd // 32, 32).permute(2, 0, 1, 3, 4).to(k_tiles.dtype)
    vt_tiles[:, :, c, :, :, q] = v.reshape(B, nkv, T, hd // 16, 16).permute(2, 0, 1, 3, 4).to(vt_tiles.dtype)


def supported(head_dim: int, max_len: int, batch: int, tokens: int) -> bool:
    """The kernel's domain: head_dim 128, one token of one sequence, and a cache length that is a
    multiple of 32 (the cache tiles' position granule)."""
    return (head_dim == HEAD_DIM and CHUNK <= max_len <= MAX_LEN and max_len % CHUNK == 0
            and batch == 1 and tokens == 1)


def decode_attention(qkv: torch.Tensor, pos: torch.Tensor, inv_freq: torch.Tensor,
                     k_cache: torch.Tensor, vt_cache: torch.Tensor, n_heads: int, n_kv: int,
                     scale: float, warm=()) -> torch.Tensor:
    """qkv [..., (n_heads + 2 n_kv) * 128] fp16 (one token); pos int64 [1]; inv_freq fp32 [64];
    k_cache [.., n_kv, L/32, 2, 4, 16, 32] and vt_cache [.., n_kv, L/32, 8, 16, 32] fp16, this
    layer's tiled caches (k_to_tiles / vt_to_tiles), updated at pos. Returns the attention output
    [1, 1, n_heads * 128] fp16. warm: tensors the launch reads into the caches for the launches
    after it, as decode_attention_ranges takes them."""
    hd = HEAD_DIM
    assert qkv.shape[-1] == (n_heads + 2 * n_kv) * hd and qkv.numel() == qkv.shape[-1]
    L = k_cache.shape[-5] * CHUNK
    assert k_cache.shape[-6:] == k_cache_shape(n_kv, L) and k_cache.numel() == n_kv * L * hd
    assert vt_cache.shape[-5:] == vt_cache_shape(n_kv, L) and vt_cache.numel() == n_kv * L * hd
    assert k_cache.is_contiguous() and vt_cache.is_contiguous()
    if qkv.dtype != torch.float16 or k_cache.dtype != torch.float16 or vt_cache.dtype != torch.float16:
        raise ValueError("decode_attention: qkv and the cache must be float16")
    if pos.dtype != torch.int64 or inv_freq.dtype != torch.float32:
        raise ValueError("decode_attention: pos int64, inv_freq float32")
    q = qkv.reshape(-1)
    if q.stride(0) != 1:
        q = q.contiguous()
    warm = _lib.warm_list(warm, "decode_attention")
    dev = _lib.require_gpu(q, pos, inv_freq, k_cache, vt_cache, *warm, what="decode_attention")
    out = torch.empty((1, 1, n_heads * hd), dtype=torch.float16, device=dev)
    freq = inv_freq.contiguous()
    wp, wb = _lib.warm_arrays(warm)
    with _lib.device_guard(dev):
        st = _lib.load().ldk_decode_attention(
            _lib.ptr(q), _lib.ptr(pos), _lib.ptr(freq), _lib.ptr(k_cache),
            _lib.ptr(vt_cache), _lib.ptr(out), n_heads, n_kv, hd, L, float(scale), wp, wb,
            len(warm), _lib.stream(dev))
    _lib.check(st, "decode_attention")
    return out


def prefill_attention(qkv: torch.Tensor, pos: torch.Tensor, inv_freq: torch.Tensor,
                      k_cache: torch.Tensor, vt_cache: torch.Tensor, n_heads: int, n_kv: int,
                      scale: float) -> torch.Tensor:
    """The prompt's attention block (ldk_prefill_attention): qkv [1, T, (n_heads + 2 n_kv) * 128]
    fp16 (the qkv projection's rows), pos int64 [T], inv_freq fp32 [64], one layer's tiled caches
    as decode_attention takes them. RoPE on q and k, k and v written into the cache at every
    pos[t], and causal grouped-query attention of token t over the cache positions 0..pos[t].
    Returns [1, T, n_heads * 128] fp16 (the reference's prompt branch, kernels/e2e/model.py:
    212-243, in two launches instead of about twenty)."""
    hd = HEAD_DIM
    width = (n_heads + 2 * n_kv) * hd
    T = pos.numel()
    assert qkv.shape[-1] == width and qkv.numel() == T * width
    L = k_cache.shape[-5] * CHUNK
    assert k_cache.shape[-6:] == k_cache_shape(n_kv, L) and k_cache.numel() == n_kv * L * hd
    assert vt_cache.shape[-5:] == vt_cache_shape(n_kv, L) and vt_cache.numel() == n_kv * L * hd
    assert k_cache.is_contiguous() and vt_cache.is_contiguous()
    if qkv.dtype != torch.float16 or k_cache.dtype != torch.float16 or vt_cache.dtype != torch.float16:
        raise ValueError("prefill_attention: qkv and the cache must be float16")
    if pos.dtype != torch.int64 or inv_freq.dtype != torch.float32:
        raise ValueError("prefill_attention: pos int64, inv_freq float32")
    rows = qkv.reshape(T, width)
    if rows.stride(1) != 1:
        rows = rows.contiguous()
    p = pos.contiguous()
    dev = _lib.require_gpu(rows, p, inv_freq, k_cache, vt_cache, what="prefill_attention")
    q_scratch = torch.empty((T, n_heads * hd), dtype=torch.float16, device=dev)
    out = torch.empty((1, T, n_heads * hd), dtype=torch.float16, device=dev)
    freq = inv_freq.contiguous()
    with _lib.device_guard(dev):
        st = _lib.load().ldk_prefill_attention(
            _lib.ptr(rows), rows.stride(0), _lib.ptr(p), T, _lib.ptr(freq), _lib.ptr(k_cache),
            _lib.ptr(vt_cache), _lib.ptr(q_scratch), _lib.ptr(out), n_heads * hd, n_heads, n_kv,
            hd, L, float(scale), _lib.stream(dev))
    _lib.check(st, "prefill_attention")
    return out


def prefill_supported(head_dim: int, max_len: int, batch: int, tokens: int) -> bool:
    """prefill_attention's domain: head_dim 128, one sequence, a cache length that is a multiple
    of 32."""
    return (head_dim == HEAD_DIM and CHUNK <= max_len <= MAX_LEN and max_len % CHUNK == 0
            and batch == 1 and 1 <= tokens <= 1 << 24)


# Most position ranges the o projection's merge takes (csrc/w4a16.hip, kAttnRanges).
MERGE_MAX_RANGES = 4
# Most byte ranges one launch warms (csrc/warm.h, kWarmMax).
WARM_MAX_RANGES = _lib.WARM_MAX_RANGES


class AttnRanges(NamedTuple):
    """The decode attention left as per-range partials in the library's device memory (see
    decode_attention_ranges): what the consumer that merges them needs to know."""

    pos: torch.Tensor
    max_len: int
    rlen: int
    n_heads: int


def ranges_len(max_len: int, max_ranges: int = MERGE_MAX_RANGES) -> int:
    """Positions per range for a cache of max_len: the shortest multiple of 32 that gives at
    most max_ranges ranges."""
    per = -(-max_len // max_ranges)
    return max(CHUNK, -(-per // CHUNK) * CHUNK)


def decode_attention_ranges(qkv: torch.Tensor, pos: torch.Tensor, inv_freq: torch.Tensor,
                            k_cache: torch.Tensor, vt_cache: torch.Tensor, n_heads: int, n_kv: int,
                            scale: float, rlen: int, warm=()) -> AttnRanges:
    """decode_attention's range kernel alone (ldk_decode_attention_ranges): the cache is split
    into ranges of rlen positions and every live range leaves its partials for a consumer that
    merges them (kernels.fused.attn_linear_rmsnorm_w4a16_matmul); no output tensor. The cache
    is updated at pos as decode_attention updates it.

    warm: up to WARM_MAX_RANGES contiguous device tensors (16-byte aligned, sizes multiples of
    16 bytes) that the same launch reads into the caches with its spare workgroups, for the
    launches after it (the next projections' weights); they change no result."""
    hd = HEAD_DIM
    assert qkv.shape[-1] == (n_heads + 2 * n_kv) * hd and qkv.numel() == qkv.shape[-1]
    L = k_cache.shape[-5] * CHUNK
    assert k_cache.shape[-6:] == k_cache_shape(n_kv, L) and k_cache.numel() == n_kv * L * hd
    assert vt_cache.shape[-5:] == vt_cache_shape(n_kv, L) and vt_cache.numel() == n_kv * L * hd
    assert k_cache.is_contiguous() and vt_cache.is_contiguous()
    if qkv.dtype != torch.float16 or k_cache.dtype != torch.float16 or vt_cache.dtype != torch.float16:
        raise ValueError("decode_attention_ranges: qkv and the cache must be float16")
    if pos.dtype != torch.int64 or inv_freq.dtype != torch.float32:
        raise ValueError("decode_attention_ranges: pos int64, inv_freq float32")
    q = qkv.reshape(-1)
    if q.stride(0) != 1:
        q = q.contiguous()
    warm = _lib.warm_list(warm, "decode_attention_ranges")
    dev = _lib.require_gpu(q, pos, inv_freq, k_cache, vt_cache, *warm, what="decode_attention_ranges")
    freq = inv_freq.contiguous()
    wp, wb = _lib.warm_arrays(warm)
    with _lib.device_guard(dev):
        st = _lib.load().ldk_decode_attention_ranges(
            _lib.ptr(q), _lib.ptr(pos), _lib.ptr(freq), _lib.ptr(k_cache), _lib.ptr(vt_cache),
            n_heads, n_kv, hd, L, int(rlen), float(scale), wp, wb, len(warm), _lib.stream(dev))
    _lib.check(st, "decode_attention_ranges")
    return AttnRanges(pos, L, int(rlen), n_heads)
