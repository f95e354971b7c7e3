"""Pins oracle.reference (kernels/reference.py restated in numpy) without retyping its formulas.

dequantize_ref: element-by-element closed form on a tiny case, and the exactness argument ((q-z)
is an exact small integer, the fp16 x fp16 product is exact in float64, so one rounding of the
float64 product must reproduce it). w4a16_ref: float64 brute-force matmul. rmsnorm_ref: hand
values (constant rows), float64 evaluation with fp16 roundings, exact residual. swiglu_ref:
float64 silu with one fp16 rounding, and known values."""

import numpy as np
import pytest

from oracle import quant
from oracle.reference import (dequantize_ref, rmsnorm_bytes, rmsnorm_ref, silu_ref, swiglu_bytes,
                              swiglu_ref, w4a16_ref)


def _quantized(N, K, seed, gs=128):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float16)
    return quant.quantize_rtn(w, gs)


def test_dequant_elementwise_tiny():
    qw, s, z = _quantized(3, 256, 0)
    deq = dequantize_ref(qw, s, z, 128)
    words = qw.view(np.uint32)
    for n in range(3):
        for k in range(256):
            q = (int(words[k // 8, n]) >> (4 * (k % 8))) & 0xF
            g = k // 128
            exact = (q - float(z[g, n])) * float(s[g, n])  # exact in float64
            assert deq[n, k] == np.float16(exact), (n, k)


def test_dequant_is_one_rounding_of_the_exact_product():
    qw, s, z = _quantized(64, 384, 1)
    deq = dequantize_ref(qw, s, z, 128)
    q = quant.unpack_int4(qw).astype(np.float64)
    exact = (q - np.repeat(z, 128, 0).astype(np.float64)) * np.repeat(s, 128, 0).astype(np.float64)
    assert np.array_equal(deq.view(np.uint16), exact.T.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("M,N,K", [(1, 16, 128), (3, 8, 256)])
def test_w4a16_ref_brute_force(M, N, K):
    rng = np.random.default_rng(2)
    qw, s, z = _quantized(N, K, 3)
    x = rng.standard_normal((M, K)).astype(np.float16)
    bias = (rng.standard_normal(N) * 0.1).astype(np.float16)
    w = dequantize_ref(qw, s, z, 128).astype(np.float64)
    ref = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            ref[m, n] = sum(float(x[m, k]) * w[n, k] for k in range(K)) + float(bias[n])
    out = w4a16_ref(x, qw, s, z, 128, bias)
    assert out.dtype == np.float32 and out.shape == (M, N)
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-5)


def test_rmsnorm_constant_row_hand_value():
    """x = c everywhere: var = c^2, normed = c / sqrt(c^2 + eps), out = w * fp16(normed)."""
    x = np.full((1, 64), 2.0, dtype=np.float16)
    w = np.full(64, 0.5, dtype=np.float16)
    out = rmsnorm_ref(x, w, 1e-6)
    normed = np.float16(2.0 / np.sqrt(4.0 + 1e-6))
    assert np.all(out == np.float16(0.5) * normed)


def test_rmsnorm_matches_float64_with_roundings():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 1536)).astype(np.float16)
    r = rng.standard_normal((5, 1536)).astype(np.float16)
    w = (1 + 0.1 * rng.standard_normal(1536)).astype(np.float16)
    out, res = rmsnorm_ref(x, w, 1e-6, residual=r)
    h = (x.astype(np.float64) + r.astype(np.float64)).astype(np.float16)  # one rounding
    assert np.array_equal(res.view(np.uint16), h.view(np.uint16))       # residual is exact
    hf = h.astype(np.float64)
    normed = (hf / np.sqrt((hf * hf).mean(-1, keepdims=True) + 1e-6)).astype(np.float16)
    ref = (w.astype(np.float64) * normed.astype(np.float64)).astype(np.float16)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(out.astype(np.float64) - ref.astype(np.float64)) <= ulp)


def test_silu_known_values_and_float64():
    g = np.array([0.0, -0.0, 1.0, -1.0, 20.0, -20.0, 3.5], dtype=np.float16)
    s = silu_ref(g)
    assert s[0] == 0 and s[4] == np.float16(20.0) and abs(float(s[5])) < 1e-7 + 5e-8
    exact = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))
    ulp = np.spacing(np.abs(exact).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(s.astype(np.float64) - exact) <= ulp)


def test_swiglu_float64():
    rng = np.random.default_rng(5)
    g = (rng.standard_normal((4, 1000)) * 3).astype(np.float16)
    u = rng.standard_normal((4, 1000)).astype(np.float16)
    out = swiglu_ref(g, u)
    gf = g.astype(np.float64)
    act = (gf / (1 + np.exp(-gf))).astype(np.float16).astype(np.float64)
    ref = (act * u.astype(np.float64)).astype(np.float16)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    # silu rounds to fp16 once (<= 1 ulp apart from float64), then one more product rounding
    assert np.all(np.abs(out.astype(np.float64) - ref.astype(np.float64)) <= 2 * ulp + 1e-7)


def test_byte_formulas_kat():
    """Byte counts quoted for configs 1 (rmsnorm.py:71-74, swiglu.py:64-65)."""
    assert rmsnorm_bytes(2048, 1536, True) == 25_168_896
    assert rmsnorm_bytes(1, 1536, True) == 15_360 and rmsnorm_bytes(1, 1536, False) == 9_216
    assert swiglu_bytes(2048, 8960) == 110_100_480 and swiglu_bytes(1, 8960) == 53_760


def test_rmsnorm_parts_consistent_with_rmsnorm_ref():
    from oracle.reference import rmsnorm_parts

    rng = np.random.default_rng(6)
    x = rng.standard_normal((3, 512)).astype(np.float16)
    r = rng.standard_normal((3, 512)).astype(np.float16)
    w = (1 + 0.1 * rng.standard_normal(512)).astype(np.float16)
    h, normed, out = rmsnorm_parts(x, w, 1e-6, r)
    ref_out, ref_h = rmsnorm_ref(x, w, 1e-6, residual=r)
    assert np.array_equal(out.view(np.uint16), ref_out.view(np.uint16))
    assert np.array_equal(h.view(np.uint16), ref_h.view(np.uint16))
    assert np.array_equal((w * normed).view(np.uint16), out.view(np.uint16))
