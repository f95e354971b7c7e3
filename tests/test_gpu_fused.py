"""The fused decode entries (kernels.fused: ldk_w4a16_rmsnorm_matmul, ldk_w4a16_swiglu_matmul,
ldk_w8a16_rmsnorm_matmul, ldk_w8a16_swiglu_matmul) against the oracle's unfused chain (kernels/reference.py:9-45: rmsnorm_ref or swiglu_ref, then
the fp32 dequantize-then-matmul) and against the library's own two-launch composition.

Bars: the north star's max-abs 2e-2 and rel-L2 1e-3 against the oracle chain; the updated
residual bit-exact (one fp16 add); SwiGLU + matmul bit-identical to swiglu_fused then
w4a16_matmul (same staged activations, same plan and reduction order); RMSNorm + matmul within
a few fp16 ulps of the composition (its staged values can differ by one ulp, the row statistic
being reduced in another order)."""

import numpy as np
import pytest
import torch

from _util import assert_north_star, bits16, to_np
from kernels.bench import cases
from kernels.fp8 import FP8, quantize_fp8, w8a16_matmul
from kernels.fused import (linear_rmsnorm_w4a16_matmul, rmsnorm_w4a16_matmul,
                           rmsnorm_w8a16_matmul, swiglu_w4a16_matmul, swiglu_w8a16_matmul,
                           w4a16_matmul_swiglu, w8a16_matmul_swiglu)
from kernels.quant import quantize_rtn
from kernels.rmsnorm import rmsnorm
from kernels.swiglu import swiglu_fused
from kernels.w4a16 import w4a16_matmul
from oracle import fp8 as of
from oracle import quant as oq
from oracle.reference import rmsnorm_ref, swiglu_ref, w4a16_ref

pytestmark = pytest.mark.gpu


def _weights(N, K, seed, bias=False):
    w, _ = cases.w4a16_case(1, N, K, seed)
    qw, s, z = quantize_rtn(w.cuda())
    b = (torch.randn(N, generator=cases.gen(seed + 1)) * 0.1).half() if bias else None
    return qw, s, z, b


def _oracle_linear(xn, qw, s, z, b):
    return w4a16_ref(xn, to_np(qw), to_np(s), to_np(z), 128, None if b is None else b.numpy())


# qkv (with bias), o, gate_up, a K with more than 4 row vectors per thread in small workgroups,
# and the quantized lm_head shape
@pytest.mark.parametrize("N,K,bias", [(2048, 1536, True), (1536, 1536, False),
                                      (17920, 1536, False), (512, 8960, False),
                                      (151936, 1536, False)])
@pytest.mark.parametrize("with_res", [True, False])
def test_rmsnorm_matmul(N, K, bias, with_res, monkeypatch):
    import kernels.fused as fused_mod

    monkeypatch.setattr(fused_mod, "FUSED_NORM_MAX_N", 1 << 30)  # the fused launch at every N
    qw, s, z, b = _weights(N, K, 11, bias)
    x, r, w = cases.rmsnorm_case(1, K, 12)
    res = r.cuda() if with_res else None
    y, res_out = rmsnorm_w4a16_matmul(x.cuda().view(1, 1, K), w.cuda(), 1e-6,
                                      None if res is None else res.view(1, 1, K), qw, s, z, 128,
                                      None if b is None else b.cuda())
    assert y.shape == (1, 1, N) and y.dtype == torch.float16
    if with_res:
        xn, h = rmsnorm_ref(x.numpy(), w.numpy(), 1e-6, residual=r.numpy())
        assert np.array_equal(bits16(res_out.view(1, K)), bits16(h))
    else:
        xn = rmsnorm_ref(x.numpy(), w.numpy(), 1e-6)
        assert res_out is None
    assert_north_star(to_np(y.view(1, N)), _oracle_linear(xn, qw, s, z, b))
    # against the library's two launches: the staged activations agree to one fp16 ulp
    if with_res:
        h2, _ = rmsnorm(x.cuda(), w.cuda(), 1e-6, residual=res)
    else:
        h2 = rmsnorm(x.cuda(), w.cuda(), 1e-6)
    y2 = w4a16_matmul(h2, qw, s, z, 128, None if b is None else b.cuda())
    d = (y.view(1, N).float() - y2.float()).abs()
    assert float(d.max()) <= 4e-3 * max(1.0, float(y2.float().abs().max())), float(d.max())


def test_rmsnorm_matmul_wide_runs_two_launches():
    """Above FUSED_NORM_MAX_N columns (the 151936-row quantized lm_head) the wrapper runs the
    norm as a launch of its own and the plain GEMV: bit-identical to those two calls."""
    import kernels.fused as fused_mod

    N, K = 151936, 1536
    assert N > fused_mod.FUSED_NORM_MAX_N
    qw, s, z, _ = _weights(N, K, 13, False)
    x, r, w = cases.rmsnorm_case(1, K, 14)
    x, r, w = x.cuda().view(1, 1, K), r.cuda().view(1, 1, K), w.cuda()
    y, h = rmsnorm_w4a16_matmul(x, w, 1e-6, r, qw, s, z, 128)
    h2, res2 = rmsnorm(x, w, 1e-6, residual=r)
    assert torch.equal(h, res2) and torch.equal(y, w4a16_matmul(h2, qw, s, z, 128))


@pytest.mark.parametrize("N,K", [(1536, 8960), (1536, 1536), (256, 8960), (4096, 2048)])
def test_swiglu_matmul(N, K):
    qw, s, z, b = _weights(N, K, 21, bias=(N == 256))
    gu = cases.swiglu_case(1, K, 22)
    y = swiglu_w4a16_matmul(gu.cuda(), qw, s, z, 128, None if b is None else b.cuda())
    act = swiglu_ref(gu[:, :K].numpy(), gu[:, K:].numpy())
    assert_north_star(to_np(y), _oracle_linear(act, qw, s, z, b))
    y2 = w4a16_matmul(swiglu_fused(gu.cuda()), qw, s, z, 128, None if b is None else b.cuda())
    assert torch.equal(y, y2)


# FP8 down projection shapes: the e2e down (K split 35 ways), small K, bias, a wide N
@pytest.mark.parametrize("N,K,bias", [(1536, 8960, False), (256, 1536, True), (2048, 768, False),
                                      (17920, 1536, True)])
def test_swiglu_w8a16_matmul(N, K, bias):
    w, _ = cases.w4a16_case(1, N, K, 41)
    wq, sc = quantize_fp8(w.cuda())
    b = (torch.randn(N, generator=cases.gen(42)) * 0.1).half().cuda() if bias else None
    gu = cases.swiglu_case(1, K, 43)
    y = swiglu_w8a16_matmul(gu.cuda(), wq, sc, bias=b)
    act = swiglu_ref(gu[:, :K].numpy(), gu[:, K:].numpy())
    ref = of.w8a16_ref(act, to_np(wq.view(torch.uint8)), to_np(sc), None if b is None else to_np(b))
    assert_north_star(to_np(y), ref)
    # same staged activations, same plan and reduction order as the two launches
    assert torch.equal(y, w8a16_matmul(swiglu_fused(gu.cuda()), wq, sc, bias=b))


# FP8 qkv (bias), o, gate_up, a K of more than 256 row vectors (the statistic's extra loop), the
# e4m3 lm_head
@pytest.mark.parametrize("N,K,bias", [(2048, 1536, True), (1536, 1536, False), (17920, 1536, False),
                                      (512, 4096, False), (151936, 1536, False)])
@pytest.mark.parametrize("with_res", [True, False])
def test_rmsnorm_w8a16_matmul(N, K, bias, with_res):
    w, _ = cases.w4a16_case(1, N, K, 51)
    wq, sc = quantize_fp8(w.cuda())
    b = (torch.randn(N, generator=cases.gen(52)) * 0.1).half().cuda() if bias else None
    x, r, wn = cases.rmsnorm_case(1, K, 53)
    r_arg = r.cuda() if with_res else None
    y, res = rmsnorm_w8a16_matmul(x.cuda(), wn.cuda(), 1e-6, r_arg, wq, sc, bias=b)
    if with_res:
        xn, h = rmsnorm_ref(x.numpy(), wn.numpy(), 1e-6, residual=r.numpy())
        assert np.array_equal(bits16(res), bits16(h))  # x + residual, one fp16 add
    else:
        xn = rmsnorm_ref(x.numpy(), wn.numpy(), 1e-6)
        assert res is None
    ref = of.w8a16_ref(xn, to_np(wq.view(torch.uint8)), to_np(sc), None if b is None else to_np(b))
    assert_north_star(to_np(y), ref)
    # the two-launch composition, within a few fp16 ulps (statistic reduced in another order)
    h2 = rmsnorm(x.cuda(), wn.cuda(), 1e-6, residual=r_arg)
    y2 = w8a16_matmul(h2[0] if with_res else h2, wq, sc, bias=b)
    d = (y.float() - y2.float()).abs()
    assert float(d.max()) <= 4e-3 * max(1.0, float(y2.float().abs().max())), float(d.max())


def test_swiglu_w8a16_rows_other_than_one_compose():
    w, _ = cases.w4a16_case(1, 512, 768, 44)
    wq, sc = quantize_fp8(w.cuda())
    gu = cases.swiglu_case(3, 768, 45).cuda()
    assert torch.equal(swiglu_w8a16_matmul(gu, wq, sc), w8a16_matmul(swiglu_fused(gu), wq, sc))


# (o projection N1 x K1) -> norm -> (N2 x N1): the Qwen2.5-1.5B pair into gate_up and into a
# biased qkv-like projection; a wide first projection (more than 256 tiles) takes the composition
@pytest.mark.parametrize("N1,K1,N2,bias2", [(1536, 1536, 17920, False), (1536, 1536, 2048, True),
                                            (1536, 2048, 8960, False), (16384, 1536, 256, False)])
def test_linear_rmsnorm_pair(N1, K1, N2, bias2):
    qw1, s1, z1, b1 = _weights(N1, K1, 61, bias=True)
    qw2, s2, z2, b2 = _weights(N2, N1, 62, bias=bias2)
    b1, b2 = b1.cuda(), (None if b2 is None else b2.cuda())
    x = cases.activations(1, K1, cases.gen(63))
    _, r, wn = cases.rmsnorm_case(1, N1, 64)
    y2, h = linear_rmsnorm_w4a16_matmul(x.cuda(), qw1, s1, z1, b1, r.cuda(), wn.cuda(), 1e-6,
                                        qw2, s2, z2, b2)
    # h: the first projection's fp16 output plus the residual, bit for bit as the composition
    y1 = w4a16_matmul(x.cuda(), qw1, s1, z1, 128, b1)
    h_ref = y1 + r.cuda()
    assert torch.equal(h.view(1, N1), h_ref.view(1, N1))
    # y2 against the oracle chain (north star) and the two-launch fused norm (a few fp16 ulps)
    xn = rmsnorm_ref(to_np(h_ref), wn.numpy(), 1e-6)
    assert_north_star(to_np(y2), _oracle_linear(xn, qw2, s2, z2, None if b2 is None else b2.cpu()))
    y2c, _ = rmsnorm_w4a16_matmul(y1, wn.cuda(), 1e-6, r.cuda(), qw2, s2, z2, 128, b2)
    d = (y2.float() - y2c.float()).abs()
    assert float(d.max()) <= 4e-3 * max(1.0, float(y2c.float().abs().max())), float(d.max())


def test_rows_other_than_one_compose():
    """Prefill rows run rmsnorm/swiglu then w4a16_matmul (same results as the two calls)."""
    qw, s, z, _ = _weights(1536, 1536, 31)
    x, r, w = cases.rmsnorm_case(5, 1536, 32)
    y, res = rmsnorm_w4a16_matmul(x.cuda(), w.cuda(), 1e-6, r.cuda(), qw, s, z)
    h, res2 = rmsnorm(x.cuda(), w.cuda(), 1e-6, residual=r.cuda())
    assert torch.equal(res, res2) and torch.equal(y, w4a16_matmul(h, qw, s, z))
    gu = cases.swiglu_case(3, 768, 33)
    qd, sd, zd, _ = _weights(1536, 768, 34)
    assert torch.equal(swiglu_w4a16_matmul(gu.cuda(), qd, sd, zd),
                       w4a16_matmul(swiglu_fused(gu.cuda()), qd, sd, zd))


def test_graph_replays_match_eager():
    """Both fused entries captured in one graph and replayed with new inputs written between the
    replays: every replay equals the eager result (the split-K workspace stays clean)."""
    qw, s, z, _ = _weights(17920, 1536, 41)
    qd, sd, zd, _ = _weights(1536, 8960, 42)
    wn = (1 + 0.1 * torch.randn(1536, generator=cases.gen(43))).half().cuda()
    x = torch.zeros(1, 1536, dtype=torch.float16, device="cuda")
    r = torch.zeros_like(x)
    y, _ = rmsnorm_w4a16_matmul(x, wn, 1e-6, r, qw, s, z)  # warm-up: allocates the workspace
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        gu, res = rmsnorm_w4a16_matmul(x, wn, 1e-6, r, qw, s, z)
        out = swiglu_w4a16_matmul(gu, qd, sd, zd)
    gen = torch.Generator(device="cuda").manual_seed(44)
    for i in range(6):
        x.copy_(torch.randn(1, 1536, device="cuda", generator=gen).half())
        r.copy_(torch.randn(1, 1536, device="cuda", generator=gen).half())
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        gu2, res2 = rmsnorm_w4a16_matmul(x, wn, 1e-6, r, qw, s, z)
        out2 = swiglu_w4a16_matmul(gu2, qd, sd, zd)
        assert torch.equal(gu, gu2) and torch.equal(res, res2) and torch.equal(out, out2), i


def test_rejects_aliased_residual_output():
    from kernels import _lib

    qw, s, z, _ = _weights(1536, 1536, 51)
    x = torch.randn(1536, device="cuda").half()
    w = torch.ones(1536, device="cuda").half()
    out = torch.empty(1536, device="cuda").half()
    ws, nb = _lib.workspace(x.device)
    st = _lib.load().ldk_w4a16_rmsnorm_matmul(
        _lib.ptr(x), _lib.ptr(x), _lib.ptr(x), _lib.ptr(w), 1e-6, _lib.ptr(qw), _lib.ptr(s),
        _lib.ptr(z), None, _lib.ptr(out), 1536, 1536, 128, ws, nb, _lib.stream(x.device))
    assert st == _lib.ERR_INVALID


def test_linear_rmsnorm_pair_column_sliced_scales_and_zeros():
    """Scales/zeros passed as column slices of wider tensors (non-contiguous): each copy must
    stay alive until its launch is enqueued, else two copies can share one freed block."""
    N1, K1, N2 = 1536, 1536, 2048
    qw1, s1, z1, b1 = _weights(2 * N1, K1, 71, bias=True)
    qw2, s2, z2, _ = _weights(2 * N2, N1, 72)
    qw1c, qw2c = qw1[:, N1:].contiguous(), qw2[:, N2:].contiguous()
    s1v, z1v, s2v, z2v = s1[:, N1:], z1[:, N1:], s2[:, N2:], z2[:, N2:]
    assert not any(t.is_contiguous() for t in (s1v, z1v, s2v, z2v))
    b1 = b1[N1:].cuda()
    x = cases.activations(1, K1, cases.gen(73)).cuda()
    _, r, wn = cases.rmsnorm_case(1, N1, 74)
    y2, h = linear_rmsnorm_w4a16_matmul(x, qw1c, s1v, z1v, b1, r.cuda(), wn.cuda(), 1e-6,
                                        qw2c, s2v, z2v, None)
    y2c, hc = linear_rmsnorm_w4a16_matmul(x, qw1c, s1v.contiguous(), z1v.contiguous(), b1,
                                          r.cuda(), wn.cuda(), 1e-6, qw2c, s2v.contiguous(),
                                          z2v.contiguous(), None)
    assert torch.equal(h, hc) and torch.equal(y2, y2c)
    xn = rmsnorm_ref(to_np(hc), wn.numpy(), 1e-6)
    assert_north_star(to_np(y2), _oracle_linear(xn, qw2c, s2v.contiguous(), z2v.contiguous(), None))


@pytest.mark.parametrize("M,N,K,bias", [(128, 17920, 1536, False), (65, 17920, 1536, False),
                                        (256, 17920, 1536, False), (512, 17920, 1536, False),
                                        (200, 8192, 1536, True), (129, 17920, 1536, False),
                                        (2048, 17920, 1536, False), (8, 17920, 1536, False)])
def test_matmul_swiglu_prefill_rows(M, N, K, bias):
    """w4a16_matmul_swiglu (ldk_w4a16_matmul_swiglu: SwiGLU in the prefill GEMM's epilogue, the g
    and u halves computed by paired column groups of one workgroup) against w4a16_matmul then
    swiglu_fused, bit for bit, at prompt rows where the plan is the prefill GEMM on 64-row tiles
    (ragged last tiles at 65, 129 and 200 rows, a bias, 2 x 64 and 4 x 64 column workgroups) and
    where it is not (2048 rows: 128-row tiles; 8 rows: the decode kernels), which compose the two
    ops; and against the oracle chain."""
    from kernels import _lib

    qw, s, z, b = _weights(N, K, 81, bias)
    b = None if b is None else b.cuda()
    x = (torch.randn(M, K, generator=cases.gen(82)) * 0.5).half().cuda()
    fused = bool(_lib.load().ldk_w4a16_matmul_swiglu_applies(M, N, K, 128))
    assert fused == (M not in (2048, 8))
    act = w4a16_matmul_swiglu(x, qw, s, z, 128, b)
    ref = swiglu_fused(w4a16_matmul(x, qw, s, z, 128, b))
    assert act.shape == (M, N // 2)
    assert np.array_equal(bits16(act), bits16(ref))
    if M <= 256:
        y = _oracle_linear(x.cpu().numpy(), qw, s, z, None if b is None else b.cpu())
        assert_north_star(to_np(act), swiglu_ref(y[:, : N // 2].astype(np.float16), y[:, N // 2:].astype(np.float16)))


@pytest.mark.parametrize("M,N,K,bias,fused", [(256, 17920, 1536, False, True), (300, 17920, 1536, True, True),
                                              (512, 17920, 1536, False, True), (1024, 8192, 1536, True, True),
                                              (128, 17920, 1536, False, False), (33, 17920, 1536, True, False),
                                              (8, 17920, 1536, False, False)])
def test_w8a16_matmul_swiglu_prefill_rows(M, N, K, bias, fused):
    """w8a16_matmul_swiglu (ldk_w8a16_matmul_swiglu, the e4m3 prefill GEMM with SwiGLU in its
    epilogue) against w8a16_matmul then swiglu_fused, bit for bit, where the plan fuses (4-wave
    tiles; ragged 300 rows, a bias) and where it composes the two ops (2-wave tiles at 33 and 128
    rows, the decode kernels at 8). The fused epilogue keeps the column scale, the bias add and
    the fp16 rounding as three steps, as the plain GEMM and the split-K reduction do."""
    from kernels import _lib

    w = (torch.randn(N, K, generator=cases.gen(91)) * 0.05).half().cuda()
    wq, sc = quantize_fp8(w)
    b = (torch.randn(N, generator=cases.gen(92)) * 0.1).half().cuda() if bias else None
    x = (torch.randn(M, K, generator=cases.gen(93)) * 0.5).half().cuda()
    assert bool(_lib.load().ldk_w8a16_matmul_swiglu_applies(M, N, K)) == fused
    act = w8a16_matmul_swiglu(x, wq, sc, b)
    ref = swiglu_fused(w8a16_matmul(x, wq, sc, bias=b))
    assert act.shape == (M, N // 2)
    assert np.array_equal(bits16(act), bits16(ref))
