"""Pins oracle.fp8 against the library routine the reference itself calls for the cast
(torch's float8_e4m3fn conversion, kernels/fp8.py:29) and the reference test's bound
(tests/test_fp8.py:26-34)."""

import numpy as np
import pytest
import torch

from oracle import fp8


def _torch_cast(v: np.ndarray) -> np.ndarray:
    return torch.from_numpy(v.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_encode_matches_torch_on_every_fp16_value():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    v = h[np.isfinite(h)].astype(np.float32)
    v = v[np.abs(v) <= 448]
    assert np.array_equal(fp8.e4m3_encode(v), _torch_cast(v))


def test_encode_matches_torch_on_random_float32():
    rng = np.random.default_rng(0)
    mags = rng.choice(np.float32([1e-4, 2e-3, 1.0, 30.0, 300.0]), 500_000)
    v = np.clip(rng.standard_normal(500_000).astype(np.float32) * mags, -448, 448).astype(np.float32)
    assert np.array_equal(fp8.e4m3_encode(v), _torch_cast(v))


def test_encode_known_answers():
    """Probed values of the cast: 447 -> 448, 0.1 -> 0.1015625, 1e-4 -> 0, ties to even."""
    assert fp8.e4m3_decode(fp8.e4m3_encode(np.float32([447.0])))[0] == 448.0
    assert fp8.e4m3_decode(fp8.e4m3_encode(np.float32([0.1])))[0] == np.float32(0.1015625)
    assert fp8.e4m3_encode(np.float32([1e-4]))[0] == 0
    # 1.0625 is halfway between 1.0 (code 0x38) and 1.125 (0x39): ties to the even code 0x38.
    assert fp8.e4m3_encode(np.float32([1.0625, 1.1875]))[0] == 0x38
    assert fp8.e4m3_encode(np.float32([1.1875]))[0] == 0x3A  # between 0x39 and 0x3A -> even
    assert fp8.e4m3_encode(np.float32([-0.0]))[0] == 0x80


def test_decode_matches_torch_all_codes():
    codes = np.array([c for c in range(256) if c & 0x7F != 0x7F], dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(fp8.e4m3_decode(codes), ref)
    assert np.isnan(fp8.e4m3_decode(np.uint8([0x7F, 0xFF]))).all()


def test_quantize_roundtrip_bound():
    """Reference tests/test_fp8.py:26-34: error <= |w|/16 + s*2^-9 + 1e-5."""
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((64, 256)) * 0.02).astype(np.float16)
    wq, s = fp8.quantize_fp8(w)
    assert wq.shape == (256, 64) and s.shape == (64,) and s.dtype == np.float16
    err = np.abs(fp8.dequantize_fp8(wq, s).astype(np.float32) - w.astype(np.float32))
    bound = np.abs(w.astype(np.float32)) / 16 + s.astype(np.float32)[:, None] * 2**-9 + 1e-5
    assert np.all(err <= bound)


def test_quantize_channel_max_maps_to_448():
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((16, 128)) * 0.02).astype(np.float16)
    wq, s = fp8.quantize_fp8(w)
    vals = np.abs(fp8.e4m3_decode(wq))
    assert np.all(vals.max(axis=0) == 448.0)  # the absmax element of each channel -> +-448


@pytest.mark.parametrize("M", [1, 4])
def test_w8a16_ref_float64(M):
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((24, 64)) * 0.02).astype(np.float16)
    wq, s = fp8.quantize_fp8(w)
    x = rng.standard_normal((M, 64)).astype(np.float16)
    deq = fp8.e4m3_decode(wq).T.astype(np.float64) * s.astype(np.float64)[:, None]
    ref = x.astype(np.float64) @ deq.astype(np.float16).astype(np.float64).T
    np.testing.assert_allclose(fp8.w8a16_ref(x, wq, s), ref, rtol=1e-5, atol=1e-5)


def test_fp8_bytes_kat():
    assert fp8.fp8_bytes(17920, 1536) + 2 * 1536 + 2 * 17920 == 27_599_872
