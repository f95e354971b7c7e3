"""The tiled KV-cache layout of the fused decode attention (kernels/attention.py) on the CPU:
the torch packers against the element offsets the kernel computes (csrc/attention.hip k_offset,
vt_offset, restated here from the layout's definition), round trips, and write_kv against
writing the logical cache then packing it."""

import pytest
import torch

from kernels import attention as A


def k_offset(p, d):
    """Offset (elements) of K at (position p, dim d) in one kv head's tiles: chunk p // 32, row
    half hb and row i such that p % 32 = 8 (i // 4) + 4 hb + i % 4, dim step d // 32."""
    q = p % 32
    i, hb = 4 * (q // 8) + q % 4, (q // 4) % 2
    return (((p // 32) * 2 + hb) * 4 + d // 32) * 512 + i * 32 + d % 32


def vt_offset(d, p):
    """Offset of V at (position p, dim d): step p // 32, dim block d // 16, row d % 16, column
    p % 32."""
    return ((p // 32) * 8 + d // 16) * 512 + (d % 16) * 32 + p % 32


def test_rows_of_a_chunk_are_a_permutation():
    rows = sorted((q // 4) % 2 * 16 + 4 * (q // 8) + q % 4 for q in range(32))
    assert rows == list(range(32))


@pytest.mark.parametrize("L", [32, 96])
def test_packers_match_the_kernel_offsets(L):
    k = torch.arange(2 * L * 128, dtype=torch.float64).reshape(2, L, 128)
    v = -torch.arange(2 * L * 128, dtype=torch.float64).reshape(2, L, 128)
    kt, vt = A.k_to_tiles(k), A.vt_to_tiles(v)
    assert kt.shape == A.k_cache_shape(2, L) and vt.shape == A.vt_cache_shape(2, L)
    kf, vf = kt.reshape(2, -1), vt.reshape(2, -1)
    for h in range(2):
        for p in range(L):
            for d in range(128):
                assert kf[h, k_offset(p, d)] == k[h, p, d]
                assert vf[h, vt_offset(d, p)] == v[h, p, d]
    assert torch.equal(A.k_from_tiles(kt), k) and torch.equal(A.v_from_tiles(vt), v)


def test_write_kv_matches_packing_the_logical_cache():
    g = torch.Generator().manual_seed(0)
    B, nkv, L, T = 1, 3, 96, 5
    k0 = torch.randn(B, nkv, L, 128, generator=g)
    v0 = torch.randn(B, nkv, L, 128, generator=g)
    kt, vt = A.k_to_tiles(k0).clone(), A.vt_to_tiles(v0).clone()
    pos = torch.tensor([0, 31, 32, 57, 95])
    k_new = torch.randn(B, nkv, T, 128, generator=g)
    v_new = torch.randn(B, nkv, T, 128, generator=g)
    A.write_kv(kt, vt, pos, k_new, v_new)
    k1, v1 = k0.clone(), v0.clone()
    k1[:, :, pos] = k_new
    v1[:, :, pos] = v_new
    assert torch.equal(kt, A.k_to_tiles(k1)) and torch.equal(vt, A.vt_to_tiles(v1))


def test_supported_needs_whole_chunks():
    assert A.supported(128, 416, 1, 1) and not A.supported(128, 392, 1, 1)
    assert not A.supported(64, 416, 1, 1) and not A.supported(128, 416, 2, 1)
