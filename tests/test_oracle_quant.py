"""Pins oracle.quant (the restatement of kernels/quant.py) without retyping its formulas.

Checks: the reference tests' known answers (tests/test_quant.py:15-18,34-35 of the reference),
round trips, hand-derived RTN results (exact grids, ties to even, clamps), the RTN error bound
(tests/test_quant.py:21-31) and brute force over a tiny group."""

import numpy as np
import pytest

from oracle import quant
from oracle.reference import dequantize_ref


def test_pack_roundtrip():
    rng = np.random.default_rng(0)
    q = rng.integers(0, 16, (64, 24)).astype(np.int32)
    packed = quant.pack_int4(q)
    assert packed.shape == (8, 24) and packed.dtype == np.int32
    assert np.array_equal(quant.unpack_int4(packed), q)


def test_pack_extremes_kat():
    """All nibbles 15 -> int32 -1 (reference tests/test_quant.py:15-18)."""
    q = np.full((16, 3), 15, dtype=np.int32)
    assert np.array_equal(quant.pack_int4(q), np.full((2, 3), -1, dtype=np.int32))
    assert np.array_equal(quant.unpack_int4(quant.pack_int4(q)), q)


def test_pack_bit_positions():
    """Nibble i of word [r, n] is q[8r+i, n] in bits 4i..4i+3 (quant.py:5-7)."""
    for i in range(8):
        q = np.zeros((8, 1), dtype=np.int32)
        q[i, 0] = 1
        assert quant.pack_int4(q)[0, 0] == np.uint32(1 << (4 * i)).view(np.int32)
    q = np.arange(8, dtype=np.int32).reshape(8, 1) + 8  # 8..15
    assert quant.pack_int4(q)[0, 0] == np.uint32(0xFEDCBA98).view(np.int32)


def test_weight_bytes_kat():
    """Reference tests/test_quant.py:34-35, and the byte counts of the four Qwen2.5-1.5B
    projections: N*K/2 packed bytes plus fp16 scales and zeros per group of 128."""
    assert quant.weight_bytes(1536, 1536) == 1536 * 1536 // 2 + 2 * 12 * 1536 * 2 == 1_253_376
    assert quant.weight_bytes(17920, 1536) == 14_622_720
    assert quant.weight_bytes(1536, 8960) == 7_311_360
    assert quant.weight_bytes(256, 1536) == 208_896


def test_rtn_exact_grid():
    """A group already on a 16-level grid quantizes to its own levels: scale = step, zero from
    the minimum, q = level index (all derivable by hand)."""
    step = np.float32(0.25)
    levels = np.arange(16, dtype=np.float32)
    col = (levels[np.arange(128) % 16] - 3) * step  # values -0.75 .. 3.0, min level 0 -> -0.75
    w = col.reshape(1, 128).astype(np.float32)
    qw, s, z = quant.quantize_rtn(w, 128)
    assert s[0, 0] == np.float32(0.25) and z[0, 0] == 3.0
    assert np.array_equal(quant.unpack_int4(qw)[:, 0], (np.arange(128) % 16).astype(np.int32))


def test_rtn_ties_to_even():
    """w/scale + zero landing exactly on k + 0.5 rounds to the even integer (torch.round)."""
    # min 0, max 15 -> scale 1, zero 0; then 2.5 -> 2, 3.5 -> 4, 0.5 -> 0, 14.5 -> 14.
    base = np.zeros(128, dtype=np.float32)
    base[0], base[1] = 0.0, 15.0
    base[2:6] = [2.5, 3.5, 0.5, 14.5]
    qw, s, z = quant.quantize_rtn(base.reshape(1, 128), 128)
    q = quant.unpack_int4(qw)[:, 0]
    assert s[0, 0] == 1.0 and z[0, 0] == 0.0
    assert list(q[:6]) == [0, 15, 2, 4, 0, 14]


def test_rtn_constant_group_clamps_scale():
    """wmax == wmin -> scale = 1e-6 (float32), zero = clamp(round(-w/1e-6), 0, 15)."""
    w = np.full((2, 128), 0.5, dtype=np.float32)
    w[1] = -3e-6
    qw, s, z = quant.quantize_rtn(w, 128)
    assert s[0, 0] == np.float32(1e-6) and s[0, 1] == np.float32(1e-6)
    assert z[0, 0] == 0.0 and z[0, 1] == 3.0  # round(3e-6 / 1e-6) = 3
    q = quant.unpack_int4(qw)
    assert np.all(q[:, 0] == 15) and np.all(q[:, 1] == 0)  # 0.5/1e-6 clamps to 15; -3+3 = 0


def test_rtn_fp16_dtype_of_scales():
    """scale/zero come back in the weight's dtype (quant.py:49): fp16 for an fp16 weight."""
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((8, 256)) * 0.02).astype(np.float16)
    qw, s, z = quant.quantize_rtn(w, 128)
    assert s.dtype == np.float16 and z.dtype == np.float16
    assert qw.shape == (32, 8) and s.shape == (2, 8)
    assert np.all((z >= 0) & (z <= 15) & (z == np.round(z)))


@pytest.mark.parametrize("N,K", [(32, 128), (40, 384)])
def test_rtn_error_bound(N, K):
    """RTN error at most half a step plus fp16 rounding (reference tests/test_quant.py:21-31)."""
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
    qw, s, z = quant.quantize_rtn(w, 128)
    deq = dequantize_ref(qw, s, z, 128)
    assert deq.shape == w.shape
    step = np.repeat(s.astype(np.float32), 128, axis=0).T
    err = np.abs(deq.astype(np.float32) - w.astype(np.float32))
    assert np.all(err <= 0.5 * step + 1e-3)


def test_rtn_brute_force_small():
    """For each group, q is the 0..15 level nearest to w on the grid (level - zero) * scale,
    found by brute force over the 16 levels (ties excluded by the random data)."""
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((6, 128)) * 0.05).astype(np.float32)
    qw, s, z = quant.quantize_rtn(w, 128)
    q = quant.unpack_int4(qw)
    for n in range(6):
        sc, ze = float(s[0, n]), float(z[0, n])
        levels = (np.arange(16) - ze) * sc
        for k in range(128):
            best = int(np.argmin(np.abs(levels - float(w[n, k]))))
            assert q[k, n] == best, (n, k)
