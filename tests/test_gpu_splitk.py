"""Cross-workgroup split-K reduction at the edges of its fixed-point range.

Partials of one output meet in a 64-bit word as fixed-point integers (2^-24 resolution) while
|p| < 2^21; larger or non-finite partials go through fp32 side slots that the finishing
workgroup adds. The reference adds fp32 partials unclamped (Triton split-K atomics,
kernels/w4a16.py:218-219,272-275), so cancelling partials beyond the fixed-point range must give
the fp32 sum, and NaN/inf must propagate as in fp32 arithmetic.

Every case is built so the fp32 sums are exact: x = 1, weights (q - z) * s with s a power of two
and integer sums below 2^24. The expected output is then exact, and a clamp, a dropped side slot
or a wrong slot index shows as a wrong value, not as a tolerance question.
"""

import numpy as np
import pytest
import torch

from _util import dev
from kernels.fp8 import w8a16_matmul
from kernels.w4a16 import w4a16_matmul
from oracle import quant as oq

pytestmark = pytest.mark.gpu

K, N = 1536, 64


def _cancelling_w4(scale: float):
    """Split 0 (rows < K/2) has weights +15s, split 1 has -15s except one row of -14s: the two
    partials are +-11520 s per unit x and the output is exactly s."""
    q = np.zeros((K, N), np.int32)
    q[: K // 2] = 15
    q[K // 2] = 1
    z = np.zeros((K // 128, N), np.float16)
    z[6:] = 15
    s = np.full((K // 128, N), scale, np.float16)
    return oq.pack_int4(q), s, z


@pytest.mark.parametrize("scale", [64.0, 1024.0])  # partials 7.4e5 (fixed point) / 1.2e7 (side slots)
@pytest.mark.parametrize("M,cfg", [(1, {"block_n": 32}), (2, {}), (4, {"MFMA": True}), (3, {"GEMV": True})])
def test_w4a16_cancelling_partials(scale, M, cfg):
    qw, s, z = _cancelling_w4(scale)
    x = np.ones((M, K), np.float16)
    args = (dev(x), dev(qw), dev(s), dev(z))
    for _ in range(3):  # the finishing workgroup leaves words and slots zeroed for the next call
        out = w4a16_matmul(*args, config={**cfg, "split_k": 2}).float().cpu().numpy()
        assert np.array_equal(out, np.full((M, N), scale, np.float32)), np.unique(out)
    # and an ordinary call after the side path sees a clean workspace
    w, xr = np.random.default_rng(1).standard_normal((N, K)).astype(np.float32) * 0.02, \
        np.random.default_rng(2).standard_normal((M, K)).astype(np.float16)
    qw2, s2, z2 = oq.quantize_rtn(w.astype(np.float16))
    a = w4a16_matmul(dev(xr), dev(qw2), dev(s2), dev(z2), config={**cfg, "split_k": 1})
    b = w4a16_matmul(dev(xr), dev(qw2), dev(s2), dev(z2), config={**cfg, "split_k": 2})
    assert (a.float() - b.float()).abs().max().item() <= 4e-3  # one fp16 ulp at |y| < 4


def test_w4a16_nan_partial_among_side_path_partials():
    """Four splits: three partials of ~7.9e6 (side slots) and one NaN partial -> NaN."""
    Kn = 2048
    q = np.full((Kn, N), 15, np.int32)
    s = np.full((Kn // 128, N), 1024.0, np.float16)
    z = np.zeros_like(s)
    x = np.ones((1, Kn), np.float16)
    x[0, 3 * Kn // 4 + 5] = np.nan
    out = w4a16_matmul(dev(x), dev(oq.pack_int4(q)), dev(s), dev(z),
                       config={"block_n": 32, "split_k": 4}).float().cpu().numpy()
    assert np.isnan(out).all()
    # the slots were zeroed by the finishing workgroup: the same weights with finite x
    x[0, 3 * Kn // 4 + 5] = 0.0
    ok = w4a16_matmul(dev(x), dev(oq.pack_int4(q)), dev(s), dev(z),
                      config={"block_n": 32, "split_k": 4}).float().cpu().numpy()
    # 2047 * 15 * 1024 = 31.4e6 exceeds fp16: +inf, as fp32 -> fp16 rounds it
    assert np.isposinf(ok).all()


def test_w4a16_opposite_infinities_give_nan():
    """+inf in split 0 and -inf in split 1 sum to NaN, as in fp32."""
    q = np.full((K, N), 15, np.int32)
    s = np.full((K // 128, N), 1.0, np.float16)
    z = np.zeros_like(s)
    x = np.ones((1, K), np.float16)
    x[0, 7] = np.inf
    x[0, K // 2 + 7] = -np.inf
    out = w4a16_matmul(dev(x), dev(oq.pack_int4(q)), dev(s), dev(z),
                       config={"block_n": 32, "split_k": 2}).float().cpu().numpy()
    assert np.isnan(out).all()


def _e4m3(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(a.astype(np.float32)).to(torch.float8_e4m3fn)


@pytest.mark.parametrize("scale", [1.0, 8.0])  # partials 3.4e5 (fixed point) / 2.8e6 (side slots)
@pytest.mark.parametrize("M,cfg", [(1, {}), (4, {"GEMV": True}), (16, {"MFMA": True})])
def test_w8a16_cancelling_partials(scale, M, cfg):
    """Split 0 rows are +448, split 1 rows -448 except one of -416: output exactly 32 * scale."""
    w = np.zeros((K, N), np.float32)
    w[: K // 2] = 448.0
    w[K // 2:] = -448.0
    w[K // 2] = -416.0
    wq = _e4m3(w).to("cuda")
    sc = torch.full((N,), scale, dtype=torch.float16, device="cuda")
    x = torch.ones((M, K), dtype=torch.float16, device="cuda")
    for _ in range(3):
        out = w8a16_matmul(x, wq, sc, config={**cfg, "split_k": 2}).float().cpu().numpy()
        assert np.array_equal(out, np.full((M, N), 32.0 * scale, np.float32)), np.unique(out)


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")  # the refused call leaves it empty
def test_workspace_first_use_under_capture_is_refused():
    """The split-K workspace is allocated by the first call on a device. A first call under graph
    capture would take it from the graph's private pool: refused with a message, before any
    launch. Made outside capture, the same call is then capturable."""
    from kernels import _lib

    x = torch.randn(1, 1536, dtype=torch.float16, device="cuda")
    qw = torch.zeros(192, 1536, dtype=torch.int32, device="cuda")
    s = torch.ones(12, 1536, dtype=torch.float16, device="cuda")
    z = torch.zeros(12, 1536, dtype=torch.float16, device="cuda")
    saved = dict(_lib._workspaces)
    _lib._workspaces.clear()
    try:
        graph = torch.cuda.CUDAGraph()
        with pytest.raises(RuntimeError, match="graph capture"):
            with torch.cuda.graph(graph):
                w4a16_matmul(x, qw, s, z)
    finally:
        _lib._workspaces.clear()
        _lib._workspaces.update(saved)
    torch.cuda.synchronize()
    y = w4a16_matmul(x, qw, s, z)  # the workspace is back: the eager call runs, and again alike
    assert torch.equal(y, w4a16_matmul(x, qw, s, z))
    torch.cuda.synchronize()
