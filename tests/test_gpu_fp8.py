"""FP8 (OCP e4m3) kernels vs the oracle: quantize and dequantize bit-exact, gfx950's hardware
e4m3 decode checked on every finite code, W8A16 matmul within the north-star tolerance."""

import numpy as np
import pytest
import torch

from _util import assert_north_star, bits16, dev, to_np
from kernels.bench import cases
from kernels.fp8 import FP8, config_for, dequantize_fp8, quantize_fp8, w8a16_matmul
from oracle import fp8 as of

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("N,K", [(17920, 1536), (1536, 8960), (64, 256)])
def test_quantize_bit_exact(N, K):
    w, _ = cases.w4a16_case(1, N, K, seed=3)
    wq, s = quantize_fp8(w.cuda())
    owq, os_ = of.quantize_fp8(w.numpy())
    assert wq.dtype == FP8 and wq.shape == (K, N) and s.dtype == torch.float16
    assert np.array_equal(to_np(wq.view(torch.uint8)), owq)
    assert np.array_equal(bits16(s), bits16(os_))


def test_quantize_fp32_and_bf16_weights():
    w = torch.randn(48, 384, generator=cases.gen(11)) * 0.03
    wq, s = quantize_fp8(w.cuda())
    owq, os_ = of.quantize_fp8(w.numpy())
    assert np.array_equal(to_np(wq.view(torch.uint8)), owq)
    assert np.array_equal(to_np(s).view(np.uint32), os_.view(np.uint32))
    wb = w.bfloat16()
    wq, s = quantize_fp8(wb.cuda())
    owq, os_ = of.quantize_fp8(wb.float().numpy())
    assert np.array_equal(to_np(wq.view(torch.uint8)), owq)
    assert torch.equal(s.cpu().view(torch.int16), torch.from_numpy(os_).bfloat16().view(torch.int16))


def test_dequantize_bit_exact():
    w, _ = cases.w4a16_case(1, 1536, 1536, seed=3)
    owq, os_ = of.quantize_fp8(w.numpy())
    out = dequantize_fp8(dev(owq).view(FP8), dev(os_))
    assert np.array_equal(bits16(out), bits16(of.dequantize_fp8(owq, os_)))


def test_hardware_decode_every_finite_code():
    """x row m = e_m and scale 1: y[m, n] = e4m3(wq[m, n]) exactly (fp16 holds every e4m3 value).
    16 rows x 256 columns cover all 254 finite codes."""
    K, N = 16, 256
    codes = ((np.arange(K)[:, None] * 16 + np.arange(N)[None, :]) % 256).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0
    x = torch.zeros(16, K, dtype=torch.float16, device="cuda")
    x[torch.arange(16), torch.arange(16)] = 1.0
    out = w8a16_matmul(x, dev(codes).view(FP8), torch.ones(N, dtype=torch.float16, device="cuda"))
    ref = of.e4m3_decode(codes).astype(np.float16)
    got = to_np(out)
    nz = ref != 0
    assert np.array_equal(bits16(got)[nz], bits16(ref)[nz])
    assert np.all(got[~nz] == 0)


def _run(M, N, K, seed=3, bias=False, config=None):
    w, x = cases.w4a16_case(M, N, K, seed)
    owq, os_ = of.quantize_fp8(w.numpy())
    b = (torch.randn(N, generator=cases.gen(seed + 50)) * 0.1).half() if bias else None
    out = w8a16_matmul(x.cuda(), dev(owq).view(FP8), dev(os_), bias=None if b is None else b.cuda(),
                       config=config)
    assert out.shape == (M, N) and out.dtype == torch.float16
    return assert_north_star(out, of.w8a16_ref(x.numpy(), owq, os_, None if b is None else b.numpy()))


@pytest.mark.parametrize("M,N,K", [(1, 64, 128), (5, 48, 96), (17, 96, 256), (2, 48, 256)])
def test_small(M, N, K):
    _run(M, N, K)


# The reference's own cases (tests/test_fp8.py:37-48): its Triton config keys, N = 40 (not a
# multiple of 16), a forced three-way split and the GEMV path with bias and a two-way split.
REF_CFG = dict(BLOCK_M=16, BLOCK_N=32, BLOCK_K=32, SPLIT_K=1, GROUP_M=8)


@pytest.mark.parametrize("M,N,K", [(1, 64, 128), (5, 40, 96), (17, 96, 256)])
def test_reference_direct_cases(M, N, K):
    _run(M, N, K, config=REF_CFG)


def test_reference_split_and_gemv_cases():
    cfg = {**REF_CFG, "SPLIT_K": 3}
    assert config_for(2, 48, 256, cfg).endswith("split_k=3")
    _run(2, 48, 256, config=cfg)
    gemv = {"GEMV": True, "BLOCK_N": 32, "BLOCK_K": 64, "SPLIT_K": 2}
    assert config_for(1, 48, 256, gemv) == "valu,block_n=32,split_k=2"
    _run(1, 48, 256, bias=True, config=gemv)


@pytest.mark.parametrize("M", [1, 2, 4, 5, 16, 17, 100])
@pytest.mark.parametrize("N,K", [(40, 96), (4, 128), (8, 64), (1000, 1024), (2044, 1536), (264, 8960)])
def test_column_tails(M, N, K):
    """N % 16 != 0 (N % 4 == 0): the VALU kernel's dword loads, the MFMA kernel's 64-column tiles
    (128 where N % 8 == 0), the 16-row blocks in place of the prefill GEMM; bias on the last
    column; the default plan, the VALU kernel forced where it takes the rows, and the MFMA kernel
    forced with a K split."""
    _run(M, N, K, bias=True)
    if M <= 16:
        _run(M, N, K, config={"GEMV": True})
    _run(M, N, K, config={"MFMA": True, "split_k": 3})


@pytest.mark.parametrize("M", [1, 2, 4, 8, 16])
def test_reference_decode_shape_8960x1536(M):
    """The reference's extra decode shape (tests/test_w4a16.py:84: N = 8960, K = 1536)."""
    _run(M, 8960, 1536)


@pytest.mark.parametrize("M", [33, 128, 2048])
@pytest.mark.parametrize("N,K", [(1536, 1536), (8960, 1536), (1536, 8960)])
def test_reference_prefill_shapes(M, N, K):
    """The reference's prefill rows (tests/test_w4a16.py:89-97) in this format."""
    _run(M, N, K)


def test_bias_and_gemv_config():
    _run(1, 48, 256, bias=True, config={"GEMV": True})
    _run(3, 64, 256, bias=True)


@pytest.mark.parametrize("block_n", [16, 32, 64, 128])
def test_block_n(block_n):
    _run(1, 1536, 1536, config={"block_n": block_n})


@pytest.mark.parametrize("M", [1, 4, 8, 16])
@pytest.mark.parametrize("name,N,K", cases.QWEN_LINEARS)
def test_config3_qwen_shapes(name, N, K, M):
    _run(M, N, K)


@pytest.mark.parametrize("M", [1, 3, 8, 9, 16])
@pytest.mark.parametrize("N,K", [(48, 96), (256, 1536), (1536, 8960), (17920 // 4, 1536)])
def test_mfma_path(M, N, K):
    """The MFMA kernel (byte transpose + exact fp8 -> fp16 + v_mfma_f32_16x16x32_f16), forced at
    every row count, ragged tiles (N=48) and K that is not a multiple of 32."""
    _run(M, N, K, config={"MFMA": True})


@pytest.mark.parametrize("split_k", [1, 2, 3, 7])
def test_mfma_split_k(split_k):
    _run(16, 1536, 1536, config={"MFMA": True, "split_k": split_k})
    _run(8, 512, 8960, bias=True, config={"MFMA": True, "split_k": split_k})


@pytest.mark.parametrize("M", [17, 33, 100, 256])
@pytest.mark.parametrize("N,K,bias", [(2048, 1536, True), (1536, 8960, False), (48, 96, True)])
def test_prefill_native_rows(M, N, K, bias):
    """Prefill rows on the MFMA kernel in 16-row blocks (grid z), row tails inside a block, the
    split-K words of each block kept apart (down splits K), bias."""
    _run(M, N, K, bias=bias, config={"prefill": "native"})


@pytest.mark.parametrize("M", [1, 4, 16, 512])
def test_reference_rows(M):
    """The reference's autotuned rows (test_fp8.py slow cases: M in {1, 4, 16, 512})."""
    _run(M, 1536, 1536, bias=True)


def test_prefill_paths_agree():
    """The prefill paths (GEMM, 16-row blocks, the library's choice) meet the bar on the same
    inputs, and an unknown path name is rejected."""
    for path in ("gemm", "blocks", "native"):
        _run(300, 2048, 1536, config={"prefill": path})
    with pytest.raises(ValueError, match="prefill"):
        _run(300, 2048, 1536, config={"prefill": "dequant"})


# ---------------------------------------------------- prefill GEMM (csrc/prefill.hip, e4m3)
@pytest.mark.parametrize("M", [17, 65, 100, 128, 256])
@pytest.mark.parametrize("N,K,bias", [(2048, 1536, True), (17920, 1536, False),
                                      (1536, 8960, False), (96, 384, True)])
def test_prefill_gemm_rows(M, N, K, bias):
    """The GEMM forced at prefill row counts: row tails inside a 64/128-row tile, bias, a column
    tile past N (N = 96), long K with a K split (down)."""
    _run(M, N, K, bias=bias, config={"prefill": "gemm"})


@pytest.mark.parametrize("M", [300, 512, 2048])
@pytest.mark.parametrize("N,K", [(2048, 1536), (1536, 1536), (17920, 1536), (1536, 8960)])
def test_prefill_reference_sizes(M, N, K):
    """The library's choice for many rows at the reference's slow-test sizes (M = 512 and 2048,
    tests/test_fp8.py) on every Qwen2.5-1.5B linear shape."""
    _run(M, N, K, bias=(N == 2048))


@pytest.mark.parametrize("block_n,split_k", [(128, 0), (256, 0), (0, 3), (256, 5)])
def test_prefill_gemm_tile_and_split_arguments(block_n, split_k):
    _run(300, 1536, 8960, config={"prefill": "gemm", "block_n": block_n, "split_k": split_k})
    _run(130, 2048, 1536, bias=True, config={"prefill": "gemm", "block_n": block_n, "split_k": split_k})


def test_prefill_gemm_one_hot_rows_exact():
    """x row m = e_k with unit scales through the GEMM: y[m, n] = e4m3(wq[k, n]) exactly, so the
    LDS row permutation, the byte transpose and the fp8 -> fp16 conversion are checked bit for
    bit on every finite code, for K rows in every position of a 64-row step."""
    K, N = 1536, 2048
    g = torch.Generator().manual_seed(8)
    codes = torch.randint(0, 256, (K, N), generator=g, dtype=torch.int64).to(torch.uint8).numpy()
    codes[(codes & 0x7F) == 0x7F] = 0
    ks = list(range(0, 64)) + [64 * 7 + 3, 1000, 1535, 777, 1024]  # 69 rows: a row tail
    x = np.zeros((len(ks), K), dtype=np.float16)
    x[np.arange(len(ks)), ks] = 1.0
    out = w8a16_matmul(dev(x), dev(codes).view(FP8), torch.ones(N, dtype=torch.float16, device="cuda"),
                       config={"prefill": "gemm"})
    ref = of.e4m3_decode(codes[ks]).astype(np.float16)
    got = to_np(out)
    nz = ref != 0
    assert np.array_equal(bits16(got)[nz], bits16(ref)[nz])
    assert np.all(got[~nz] == 0)


def test_prefill_gemm_32_row_tiles_with_tail():
    """qkv-like short K at about 500 rows runs 32-row tiles on two column groups and two K
    groups; 500 rows leave a partial last row tile."""
    _run(500, 2048, 1536, bias=True, config={"prefill": "gemm"})
    _run(512, 1536, 1536, config={"prefill": "gemm"})


def test_prefill_gemm_long_k_row_tiles_fast_with_tail():
    """Long K with 16 row tiles (row tiles on the grid's fast axis), a partial last row tile."""
    _run(2000, 1536, 8960, bias=True, config={"prefill": "gemm"})


def test_prefill_gemm_two_k_groups_odd_steps():
    """Two K groups in a workgroup over 33 K-steps of 64 (17 and 16: the second group takes one
    barrier-only step), a partial last column tile (N = 1008), row tails."""
    _run(300, 1008, 2112, config={"prefill": "gemm"})
    _run(2048, 1008, 2112, bias=True, config={"prefill": "gemm"})


def test_prefill_gemm_strided_rows():
    w, x = cases.w4a16_case(150, 1536, 768, 21)
    owq, os_ = of.quantize_fp8(w.numpy())
    wide = torch.zeros(150, 1024, dtype=torch.float16)
    wide[:, 100:868] = x
    xs = wide.cuda()[:, 100:868]
    assert xs.stride(0) == 1024
    out = w8a16_matmul(xs, dev(owq).view(FP8), dev(os_), config={"prefill": "gemm"})
    assert_north_star(out, of.w8a16_ref(x.numpy(), owq, os_, None))


def test_prefill_gemm_k_split_deterministic_and_leaves_workspace_clean():
    """Long K (down at 512 rows) splits K over workgroups; the partials are summed in split order
    (same bits every call) and zeroed, so a decode split-K call right after sees a clean
    workspace."""
    w, x = cases.w4a16_case(512, 1536, 8960, 22)
    owq, os_ = of.quantize_fp8(w.numpy())
    args = (x.cuda(), dev(owq).view(FP8), dev(os_))
    outs = [w8a16_matmul(*args, config={"prefill": "gemm"}) for _ in range(3)]
    assert all(torch.equal(o, outs[0]) for o in outs[1:])
    assert_north_star(outs[0], of.w8a16_ref(x.numpy(), owq, os_, None))
    x1 = x[:1].contiguous()
    y1 = w8a16_matmul(x1.cuda(), *args[1:], config={"split_k": 5})
    assert_north_star(y1, of.w8a16_ref(x1.numpy(), owq, os_, None))


def test_prefill_gemm_rejects_k_not_multiple_of_64():
    """K = 96 has no whole 64-deep step: forcing the GEMM is an error, the library's choice
    keeps the 16-row blocks."""
    w, x = cases.w4a16_case(100, 48, 96, 4)
    owq, os_ = of.quantize_fp8(w.numpy())
    with pytest.raises(RuntimeError, match="prefill GEMM"):
        w8a16_matmul(x.cuda(), dev(owq).view(FP8), dev(os_), config={"prefill": "gemm"})
    _run(100, 48, 96)


def test_mfma_one_hot_rows_exact():
    """x row m = e_{3m}: the MFMA path returns e4m3(wq[3m, n]) * scale exactly (one product,
    one rounding), so the in-register byte transpose and the decode are checked bit for bit."""
    K, N = 64, 384
    g = torch.Generator().manual_seed(5)
    codes = torch.randint(0, 256, (K, N), generator=g, dtype=torch.int64).to(torch.uint8).numpy()
    codes[(codes & 0x7F) == 0x7F] = 0
    x = torch.zeros(16, K, dtype=torch.float16, device="cuda")
    x[torch.arange(16), torch.arange(16) * 3] = 1.0
    out = w8a16_matmul(x, dev(codes).view(FP8), torch.ones(N, dtype=torch.float16, device="cuda"),
                       config={"MFMA": True})
    ref = of.e4m3_decode(codes[::3][:16]).astype(np.float16)
    assert np.array_equal(bits16(to_np(out)) & 0x7FFF | (bits16(ref) & 0x8000) * (ref != 0),
                          bits16(ref) & 0x7FFF | (bits16(ref) & 0x8000) * (ref != 0))


# ---------------------------------------------------------------- decode rows through the library's plan
@pytest.mark.parametrize("M", [2, 3, 4, 5, 8, 9, 16])
@pytest.mark.parametrize("N,K", [(17920, 1536), (2048, 1536), (1536, 1536), (256, 1536), (1536, 8960),
                                 (1040, 512), (48, 96)])
def test_decode_rows_default_plan(M, N, K):
    """Decode rows 2-16 on the library's choice (the MFMA kernel: 128-column tiles over all of K
    on gate_up, 64-column tiles split into K pieces on the narrower shapes), on the Qwen shapes,
    a column tail (N = 1040) and short K, against the oracle."""
    _run(M, N, K)


def test_decode_rows_bias_strided_and_unaligned_rows():
    """Bias; x as a row-strided view (ldx > K); x not 16-byte aligned."""
    _run(7, 2048, 1536, bias=True)
    w, x = cases.w4a16_case(6, 1024, 768, 7)
    owq, os_ = of.quantize_fp8(w.numpy())
    ref = of.w8a16_ref(x.numpy(), owq, os_, None)
    big = torch.zeros(6, 1024, dtype=torch.float16, device="cuda")
    big[:, :768] = x.cuda()
    assert_north_star(w8a16_matmul(big[:, :768], dev(owq).view(FP8), dev(os_)), ref)
    off = torch.zeros(6 * 768 + 1, dtype=torch.float16, device="cuda")
    xv = off[1:].view(6, 768)
    xv.copy_(x.cuda())
    assert_north_star(w8a16_matmul(xv, dev(owq).view(FP8), dev(os_)), ref)


def test_mfma_every_code_exact():
    """x row m = e_k and scale 1 through the MFMA kernel at K = 32: y[m, n] = e4m3(wq[k, n])
    exactly for every finite code (32 rows x 256 columns hold them all)."""
    K, N = 32, 256
    codes = ((np.arange(K)[:, None] * 16 + np.arange(N)[None, :] * 7) % 256).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0
    wq = dev(codes).view(FP8)
    ones = torch.ones(N, dtype=torch.float16, device="cuda")
    for k0 in (0, 16):
        x = torch.zeros(16, K, dtype=torch.float16, device="cuda")
        x[torch.arange(16), k0 + torch.arange(16)] = 1.0
        got = to_np(w8a16_matmul(x, wq, ones))
        ref = of.e4m3_decode(codes[k0:k0 + 16]).astype(np.float16)
        nz = ref != 0
        assert np.array_equal(bits16(got)[nz], bits16(ref)[nz]), k0
        assert np.all(got[~nz] == 0)


@pytest.mark.parametrize("M", [3, 4, 16, 17, 40])
@pytest.mark.parametrize("N,K", [(17920, 1536), (1536, 8960), (208, 1536), (2064, 512)])
def test_mfma_64_column_tiles(M, N, K):
    """The MFMA kernel on 64-column tiles (block_n 64): tile pairs sharing a line are placed on
    one XCD through the workgroup order, the tiles past the last group of 16 keep their index
    (2064 columns: 33 tiles, the last one ragged)."""
    _run(M, N, K, config={"MFMA": True, "block_n": 64})


def test_mfma_64_column_tiles_every_code_exact():
    """One-hot rows through the 64-column MFMA kernel reproduce every finite code exactly."""
    K, N = 32, 256
    codes = ((np.arange(K)[:, None] * 16 + np.arange(N)[None, :] * 7) % 256).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0
    wq = dev(codes).view(FP8)
    ones = torch.ones(N, dtype=torch.float16, device="cuda")
    for k0 in (0, 16):
        x = torch.zeros(16, K, dtype=torch.float16, device="cuda")
        x[torch.arange(16), k0 + torch.arange(16)] = 1.0
        got = to_np(w8a16_matmul(x, wq, ones, config={"MFMA": True, "block_n": 64}))
        ref = of.e4m3_decode(codes[k0:k0 + 16]).astype(np.float16)
        nz = ref != 0
        assert np.array_equal(bits16(got)[nz], bits16(ref)[nz]), k0
        assert np.all(got[~nz] == 0)


# ------------------------------------------------------- prefill rows on the 16-row blocks (plan)
@pytest.mark.parametrize("M", [17, 40, 64, 65, 100, 160])
@pytest.mark.parametrize("N,K", [(1536, 1536), (2048, 1536), (1536, 8960), (1000, 1536), (2064, 512),
                                 (1536, 1000), (1536, 2600)])
def test_prefill_row_blocks_default_plan(M, N, K):
    """The library's choice at prefill rows: short K on 64-column 16-row blocks with K split toward
    256 workgroups (16 waves where split), long K on 128-column blocks in at least two splits, the
    prefill GEMM past where the blocks fit; ragged last row block, N % 8 != 0 (1000), K not a
    multiple of the 32-row K step (1000) and long K not a multiple of 64 (2600)."""
    _run(M, N, K, bias=(N == 2048))


def test_prefill_row_blocks_one_hot_rows_exact():
    """16-wave 64-column blocks with K split at prefill rows (M = 40, K = 1536: 3 row blocks in
    three splits): one-hot x rows return e4m3(wq[k, n]) * scale exactly, so the split words, the
    row blocks and the 16-wave reduction are checked bit for bit."""
    M, K, N = 40, 1536, 1536
    g = torch.Generator().manual_seed(6)
    codes = torch.randint(0, 256, (K, N), generator=g, dtype=torch.int64).to(torch.uint8).numpy()
    codes[(codes & 0x7F) == 0x7F] = 0
    ks = (torch.arange(M) * 37) % K
    x = torch.zeros(M, K, dtype=torch.float16, device="cuda")
    x[torch.arange(M), ks.cuda()] = 1.0
    assert config_for(M, N, K) == "mfma,block_n=64,split_k=3"
    out = w8a16_matmul(x, dev(codes).view(FP8), torch.ones(N, dtype=torch.float16, device="cuda"))
    ref = of.e4m3_decode(codes[ks.numpy()]).astype(np.float16)
    assert np.array_equal(bits16(to_np(out)) & 0x7FFF | (bits16(ref) & 0x8000) * (ref != 0),
                          bits16(ref) & 0x7FFF | (bits16(ref) & 0x8000) * (ref != 0))
