"""The one-row fp16 GEMV of the tied lm_head (`ldk_f16_gemv`, kernels.head.lm_head) against a
float64 CPU product of the same fp16 operands (the reference's `F.linear(h, self.lm_head)`,
kernels/e2e/model.py:253, with fp32-or-better accumulation).

Tolerance: the north star's bound for fp16 outputs of an fp32-accumulated product, max-abs 2e-2
and relative L2 1e-3 (the only error past the exact sum is fp32 accumulation and the final fp16
rounding); on top, 99.9% of outputs must lie within one fp16 ulp of the float64 result."""

import numpy as np
import pytest
import torch

from kernels.head import applies, lm_head
from _util import assert_north_star

pytestmark = pytest.mark.gpu


def _case(N, K, seed, ldw=None):
    g = torch.Generator().manual_seed(seed)
    ldw = ldw or K
    wfull = (torch.randn(N, ldw, generator=g) * 0.02).half()
    w = wfull[:, :K]
    h = torch.randn(1, 1, K, generator=g).half()
    ref = (w.double() @ h.reshape(K).double()).reshape(1, 1, N)
    return h, wfull, w, ref


def _check(out, ref):
    assert out.dtype == torch.float16 and out.shape == ref.shape
    o = out.float().cpu().double()
    assert_north_star(o.numpy(), ref.numpy())
    # one fp16 ulp of the float64 result bounds fp32 accumulation + one rounding; allow 0.1% of
    # outputs past it (a product with an fp16 subnormal weight may round differently)
    _, e = torch.frexp(ref.half().float())
    ulp = torch.pow(2.0, torch.clamp(e.double() - 11, min=-24))
    far = ((o - ref).abs() > ulp).double().mean().item()
    assert far <= 1e-3, far


@pytest.mark.parametrize("rpw", [0, 4, 8])
@pytest.mark.parametrize("N,K", [(1, 8), (7, 1536), (1001, 1536), (4099, 520), (333, 512), (65, 1024),
                                 (2049, 2048), (31, 8)])
def test_matches_float64(N, K, rpw):
    h, _, w, ref = _case(N, K, seed=N * 7 + K)
    wd = w.contiguous().cuda()
    assert applies(h.cuda(), wd)
    _check(lm_head(h.cuda(), wd, rows_per_wave=rpw), ref)


def test_strided_table():
    """A row stride past K (a view of a wider table), as a tied embedding slice could be."""
    h, wfull, w, ref = _case(777, 1536, seed=5, ldw=1544)
    wv = wfull.cuda()[:, :1536]
    assert wv.stride(0) == 1544
    _check(lm_head(h.cuda(), wv), ref)


@pytest.mark.slow
def test_qwen_lm_head_shape():
    """The config-4 table: 151936 x 1536 (466.7 MB)."""
    h, _, w, ref = _case(151936, 1536, seed=4)
    _check(lm_head(h.cuda(), w.contiguous().cuda()), ref)


def test_graph_replay_matches_eager():
    h, _, w, ref = _case(4096, 1536, seed=9)
    hd, wd = h.cuda(), w.contiguous().cuda()
    eager = lm_head(hd, wd)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g):
            out = lm_head(hd, wd)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(3):
        hd.copy_((h * (i + 1)).cuda())
        g.replay()
        torch.cuda.synchronize()
        want = lm_head(hd, wd)
        torch.cuda.synchronize()
        assert torch.equal(out, want)
    hd.copy_(h.cuda())
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, eager)


def test_rejects_what_it_does_not_cover():
    w = torch.zeros(16, 12, dtype=torch.float16, device="cuda")
    h = torch.zeros(1, 12, dtype=torch.float16, device="cuda")
    assert not applies(h, w)
    with pytest.raises(ValueError):
        lm_head(h, w)  # K not a multiple of 8
    w = torch.zeros(16, 16, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        lm_head(torch.zeros(2, 16, dtype=torch.float16, device="cuda"), w)  # two rows
    with pytest.raises(ValueError):
        lm_head(torch.zeros(1, 16, dtype=torch.float32, device="cuda"), w)
    w = torch.zeros(4, 2056, dtype=torch.float16, device="cuda")
    h = torch.zeros(1, 2056, dtype=torch.float16, device="cuda")
    assert not applies(h, w)
    with pytest.raises(RuntimeError):
        lm_head(h, w)  # K > 2048: LDK_ERR_UNSUPPORTED
    with pytest.raises(ValueError):
        lm_head(torch.zeros(1, 16, dtype=torch.float16, device="cuda"),
                torch.zeros(4, 16, dtype=torch.float16, device="cuda"), rows_per_wave=3)


@pytest.mark.parametrize("with_res", [False, True])
@pytest.mark.parametrize("N,K,rpw", [(1001, 1536, 0), (4099, 520, 8), (65, 2048, 4), (151936, 1536, 0)])
def test_fused_rmsnorm_head(N, K, rpw, with_res):
    """x = rmsnorm(h (+ residual)) * w formed inside the head launch, against the oracle's
    rmsnorm_ref (numpy, the reference's rounding steps) followed by a float64 product. The
    staged x may differ from the oracle's by an fp16 ulp where the row statistic's fp32 sum order
    tips a rounding, so the bar is the north star's fp16-output bound."""
    from oracle.reference import rmsnorm_ref

    g = torch.Generator().manual_seed(N + K + with_res)
    w = (torch.randn(N, K, generator=g) * 0.02).half()
    h = torch.randn(1, 1, K, generator=g).half()
    res = torch.randn(1, 1, K, generator=g).half() if with_res else None
    nw = (1 + 0.1 * torch.randn(K, generator=g)).half()
    xn = rmsnorm_ref(h.numpy(), nw.numpy(), 1e-6, residual=None if res is None else res.numpy())
    xn = xn[0] if with_res else xn
    ref = (w.double() @ torch.from_numpy(np.ascontiguousarray(xn)).reshape(K).double()).reshape(1, 1, N)
    out = lm_head(h.cuda(), w.contiguous().cuda(), rows_per_wave=rpw, norm_weight=nw.cuda(), eps=1e-6,
                  residual=None if res is None else res.cuda())
    assert out.shape == (1, 1, N) and out.dtype == torch.float16
    assert_north_star(out.float().cpu().double().numpy(), ref.numpy())
    # the fused launch equals the unfused pair (standalone RMSNorm kernel, then the head) to fp16
    # output tolerance
    from kernels.rmsnorm import rmsnorm

    xr = rmsnorm(h.cuda(), nw.cuda(), 1e-6, None if res is None else res.cuda())
    xr = xr[0] if with_res else xr
    two = lm_head(xr, w.contiguous().cuda(), rows_per_wave=rpw)
    d = (out.float() - two.float()).abs().max().item()
    assert d <= 2e-2, d


def test_fused_rmsnorm_head_rejects():
    w = torch.zeros(16, 16, dtype=torch.float16, device="cuda")
    h = torch.zeros(1, 16, dtype=torch.float16, device="cuda")
    with pytest.raises(ValueError):
        lm_head(h, w, residual=h)  # residual without a norm weight
    with pytest.raises(ValueError):
        lm_head(h, w, norm_weight=torch.zeros(8, dtype=torch.float16, device="cuda"))
