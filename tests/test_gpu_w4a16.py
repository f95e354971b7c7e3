"""W4A16 HIP kernels vs the oracle's fp32 dequantize-then-matmul (kernels/reference.py:39-45) on
the same seeded inputs, through the C ABI. Acceptance (north star): max-abs <= 2e-2 and
relative-L2 <= 1e-3 against the fp32 reference; dequantized weights bit-exact (checked directly
by the one-hot tests: x = e_k returns column k of the dequantized weight exactly)."""

import numpy as np
import pytest
import torch

from _util import assert_north_star, bits16, dev, to_np
from kernels.bench import cases
from kernels.cuda.w4a16_cuda import w4a16_decode_cuda
from kernels.w4a16 import config_for, kernel_name, w4a16_matmul
from oracle import quant as oq
from oracle.reference import dequantize_ref, w4a16_ref

pytestmark = pytest.mark.gpu


def _make(M, N, K, seed, gs=128, bias=False):
    w, x = cases.w4a16_case(M, N, K, seed)
    qw, s, z = oq.quantize_rtn(w.numpy(), gs)
    b = (torch.randn(N, generator=cases.gen(seed + 100)) * 0.1).half().numpy() if bias else None
    return x.numpy(), qw, s, z, b


def _run(M, N, K, seed=2, gs=128, bias=False, config=None, entry=w4a16_matmul):
    x, qw, s, z, b = _make(M, N, K, seed, gs, bias)
    out = entry(dev(x), dev(qw), dev(s), dev(z), gs, bias=None if b is None else dev(b),
                **({"config": config} if config is not None else {}))
    assert out.shape == (M, N) and out.dtype == torch.float16
    return assert_north_star(out, w4a16_ref(x, qw, s, z, gs, b))


# ---------------------------------------------------------------- reference test shapes
@pytest.mark.parametrize("M,N,K", [(1, 64, 256), (3, 40, 128), (17, 96, 384), (5, 64, 256)])
def test_small(M, N, K):
    _run(M, N, K)


def test_bias():
    _run(1, 64, 256, bias=True)
    _run(4, 64, 256, bias=True)


@pytest.mark.parametrize("factored", [True, False])
@pytest.mark.parametrize("N,K", [(64, 256), (40, 384), (96, 128)])
def test_gemv_modes(N, K, factored):
    _run(1, N, K, config={"GEMV": True, "FACTORED": factored})


@pytest.mark.parametrize("block_n", [16, 32, 64])
def test_block_n_variants(block_n):
    _run(1, 1536, 1536, config={"block_n": block_n})
    _run(4, 1536, 1536, config={"block_n": block_n})


@pytest.mark.parametrize("split_k", [1, 2, 3, 4, 12])
def test_split_k_variants(split_k):
    """Cross-workgroup split of K (partials meet in the workspace; the last workgroup reduces)."""
    _run(1, 1536, 1536, config={"block_n": 32, "split_k": split_k})
    _run(2, 1536, 1536, config={"split_k": split_k})
    _run(3, 1536, 1536, config={"split_k": split_k})
    _run(16, 1536, 1536, config={"split_k": split_k})


@pytest.mark.parametrize("cpw", [1, 2, 4])
def test_chunks_per_wave_variants(cpw):
    """Several load chunks in flight per wave (rounds of cpw chunks, runtime loop over rounds),
    with and without a cross-workgroup split, ragged chunk counts included (K=8960: 70 groups)."""
    for bn in (16, 32, 64):
        _run(1, 1536, 8960, config={"block_n": bn, "chunks_per_wave": cpw})
        _run(1, 512, 8960, config={"block_n": bn, "chunks_per_wave": cpw, "split_k": 3})
    _run(1, 17920 // 8, 1536, config={"chunks_per_wave": cpw})
    if cpw <= 2:
        for M in (2, 3, 4):
            _run(M, 1536, 8960, config={"chunks_per_wave": cpw, "block_n": 32})
        _run(16, 1536, 8960, config={"chunks_per_wave": cpw})
        _run(12, 512, 8960, config={"chunks_per_wave": cpw, "split_k": 5})
        _run(4, 512, 1536, config={"MFMA": True, "chunks_per_wave": cpw})


@pytest.mark.parametrize("gs", [32, 256])
def test_chunks_per_wave_group_sizes(gs):
    _run(1, 512, 4096, gs=gs, config={"chunks_per_wave": 2})
    _run(16, 512, 4096, gs=gs, config={"chunks_per_wave": 2})


def test_split_k_repeated_calls_keep_counters_clean():
    """The last workgroup of a tile resets its counter: many calls in a row stay correct."""
    x, qw, s, z, _ = _make(1, 1536, 8960, 7)
    ref = w4a16_ref(x, qw, s, z)
    args = (dev(x), dev(qw), dev(s), dev(z))
    for _ in range(20):
        out = w4a16_matmul(*args, config={"split_k": 7})
    torch.cuda.synchronize()
    assert_north_star(out, ref)


def test_split_k_deterministic():
    """Split partials meet as fixed-point integers: any arrival order gives the same bits."""
    x, qw, s, z, _ = _make(4, 1536, 8960, 11)
    args = (dev(x), dev(qw), dev(s), dev(z))
    for cfg in ({"split_k": 7}, {"split_k": 5, "MFMA": True}):
        outs = [w4a16_matmul(*args, config=cfg) for _ in range(8)]
        for o in outs[1:]:
            assert torch.equal(o, outs[0])


def test_split_k_nonfinite_input_propagates():
    """An inf in x makes every output non-finite on the split path, as on the unsplit one."""
    x, qw, s, z, _ = _make(1, 256, 2048, 12)
    x = x.copy()
    x[0, 5] = np.inf
    args = (dev(x), dev(qw), dev(s), dev(z))
    a = w4a16_matmul(*args, config={"split_k": 1})
    b = w4a16_matmul(*args, config={"split_k": 4})
    assert not torch.isfinite(a).any() and not torch.isfinite(b).any()


def test_split_k_large_partials():
    """Partial sums of magnitude ~1e4 (outputs near the fp16 limit) stay within tolerance."""
    x, qw, s, z, _ = _make(2, 512, 8960, 13)
    s = (s.astype(np.float32) * 160).astype(np.float16)
    out = w4a16_matmul(dev(x * 4), dev(qw), dev(s), dev(z), config={"split_k": 6})
    ref = w4a16_ref(x * 4, qw, s, z)
    assert 1e3 < np.abs(ref).max() < 6e4
    got = out.float().cpu().numpy()
    assert np.all(np.abs(got - ref) <= 2e-3 * np.abs(ref) + 0.5)


@pytest.mark.parametrize("M,N", [(16, 17920), (9, 17920), (4, 17920), (16, 2048), (3, 4100),
                                 (16, 260)])
@pytest.mark.parametrize("block_n", [32, 64, 128])
def test_mfma_tile_widths(M, N, block_n):
    """The MFMA kernel's 32-column tiles (8-byte loads, two MFMA column tiles per lane), 64- and
    128-column tiles (one or two 16-byte line halves per lane, four or eight MFMA column tiles),
    including column tails that end inside a tile."""
    _run(M, N, 1536, config={"MFMA": True, "block_n": block_n})


def test_mfma_32_column_tiles_split_and_prefill():
    """32-column MFMA tiles with the cross-workgroup K split (down projection) and in prefill
    row blocks (16 rows at M = 40: 64 tiles x 3 blocks), with bias."""
    _run(8, 1536, 8960, bias=True, config={"MFMA": True, "block_n": 32})
    _run(16, 1536, 8960, config={"MFMA": True, "block_n": 32, "split_k": 7})
    _run(40, 2048, 1536, bias=True, config={"MFMA": True, "block_n": 32})


def test_mfma_split_k_with_128_columns():
    _run(16, 1536, 8960, config={"MFMA": True, "block_n": 128, "split_k": 5})
    _run(7, 512, 8960, config={"MFMA": True, "block_n": 128, "split_k": 14}, bias=True)


@pytest.mark.parametrize("M", [1, 4, 9, 16])
def test_mfma_and_valu_paths_agree_with_reference(M):
    if M <= 8:
        _run(M, 2048, 1536, config={"MFMA": True})
        _run(M, 2048, 1536, config={"GEMV": True})
    else:
        _run(M, 2048, 1536, config={"MFMA": True})


@pytest.mark.parametrize("gs", [32, 64, 256])
def test_group_sizes(gs):
    _run(1, 256, 1024, gs=gs)
    _run(2, 256, 1024, gs=gs)
    _run(16, 256, 1024, gs=gs)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 7, 8, 9, 12, 16])
def test_all_decode_rows(M):
    _run(M, 1536, 1536)


def test_odd_n_and_bias():
    _run(5, 1000, 1024, bias=True)
    _run(1, 132, 256, bias=True)
    for M in (1, 2, 4, 16):  # the reference's odd N = 200 with bias (test_w4a16.py slow cases)
        _run(M, 200, 1536, bias=True)


@pytest.mark.parametrize("M", [33, 128, 2048])
@pytest.mark.parametrize("N,K", [(1536, 1536), (256, 1536)])
def test_prefill_reference_rows(M, N, K):
    """The reference's prefill rows (test_w4a16.py slow cases: M in {33, 128, 2048}): the native
    MFMA blocks up to 256 rows, dequantize + hipBLASLt beyond."""
    _run(M, N, K, bias=True)


def test_3d_input():
    x, qw, s, z, _ = _make(6, 32, 128, 3)
    out = w4a16_matmul(dev(x).view(2, 3, 128), dev(qw), dev(s), dev(z))
    assert out.shape == (2, 3, 32)
    assert_north_star(out.view(6, 32), w4a16_ref(x, qw, s, z))


def test_strided_rows():
    """x given as a row-strided view (ldx > K) is handled without a copy."""
    x, qw, s, z, _ = _make(4, 256, 512, 4)
    big = torch.zeros(4, 1024, dtype=torch.float16, device="cuda")
    big[:, :512] = dev(x)
    out = w4a16_matmul(big[:, :512], dev(qw), dev(s), dev(z))
    assert_north_star(out, w4a16_ref(x, qw, s, z))


# ---------------------------------------------------------------- exactness of the unpacking
@pytest.mark.parametrize("factored", [True, False])
def test_one_hot_rows_reproduce_dequantized_weight(factored):
    """x = e_k: the output is column k of dequant(W), exactly (every product and sum is exact).
    Checks the nibble order, the x pairing and the per-group scale/zero for every k."""
    N, K = 256, 512
    _, qw, s, z, _ = _make(1, N, K, 9)
    deq = dequantize_ref(qw, s, z, 128)  # [N, K] fp16
    qwd, sd, zd = dev(qw), dev(s), dev(z)
    for k0 in range(0, K, 16):
        rows = []
        for k in range(k0, k0 + 16):
            x = torch.zeros(1, K, dtype=torch.float16, device="cuda")
            x[0, k] = 1.0
            rows.append(w4a16_matmul(x, qwd, sd, zd, config={"FACTORED": factored}))
        got = torch.cat(rows).cpu().numpy()
        assert np.array_equal(bits16(got), bits16(np.ascontiguousarray(deq[:, k0:k0 + 16].T))), k0


def test_two_rows_factored_paths():
    """M = 2 runs the factored VALU kernel with two x rows per pass: whole tiles, the gate_up
    hybrid (one-wave split pieces), the down projection's LDS-reduced split, bias, strided rows."""
    _run(2, 17920, 1536, bias=True)
    _run(2, 1536, 8960, bias=True)
    _run(2, 2048, 1536, bias=True)
    for bn in (16, 32, 64):
        _run(2, 1000, 1024, config={"block_n": bn})
    x, qw, s, z, _ = _make(2, 256, 512, 4)
    big = torch.zeros(2, 1024, dtype=torch.float16, device="cuda")
    big[:, :512] = dev(x)
    assert_north_star(w4a16_matmul(big[:, :512], dev(qw), dev(s), dev(z)), w4a16_ref(x, qw, s, z))


@pytest.mark.parametrize("N,K", [(256, 512), (1536, 8960)])
def test_two_rows_one_hot_reproduce_dequantized_weight(N, K):
    """Two rows e_j, e_k: both output rows are exact columns of dequant(W), through whole tiles
    (256 x 512) and the cross-workgroup split (1536 x 8960)."""
    _, qw, s, z, _ = _make(1, N, K, 9)
    deq = dequantize_ref(qw, s, z, 128)
    qwd, sd, zd = dev(qw), dev(s), dev(z)
    for j, k in ((0, 1), (7, K - 1), (K // 2 + 3, 129), (K - 8, 8)):
        x = torch.zeros(2, K, dtype=torch.float16, device="cuda")
        x[0, j] = 1.0
        x[1, k] = 1.0
        got = w4a16_matmul(x, qwd, sd, zd).cpu().numpy()
        assert np.array_equal(bits16(got), bits16(np.ascontiguousarray(deq[:, [j, k]].T))), (j, k)


def test_one_hot_multi_row():
    """M = 16 rows, row m = e_m: the exact path returns dequantized weights too."""
    N, K = 128, 256
    _, qw, s, z, _ = _make(1, N, K, 10)
    deq = dequantize_ref(qw, s, z, 128)
    x = torch.zeros(16, K, dtype=torch.float16, device="cuda")
    x[torch.arange(16), torch.arange(16) * 3] = 1.0
    out = w4a16_matmul(x, dev(qw), dev(s), dev(z))
    assert np.array_equal(bits16(out), bits16(np.ascontiguousarray(deq[:, ::3][:, :16].T)))


# ---------------------------------------------------------------- MFMA kernel with x staged in LDS
@pytest.mark.parametrize("M", [3, 4, 5, 8, 9, 12, 16])
@pytest.mark.parametrize("N,K", [(17920, 1536), (2048, 1536), (1536, 1536), (1024, 512), (256, 1536),
                                 (200, 1536), (4100, 1280)])
def test_mfma_x_rows(M, N, K):
    """Decode rows on the x-staged MFMA kernel: row tiles of 4/8/16 with rows past M staged as
    zeros, twelve waves of one group, six of two (gate_up at <= 4 rows) and six of one (K = 512:
    four groups, two waves idle; K = 1280: ten groups, two waves idle); column tails inside a
    32-column tile (N = 200, 4100)."""
    from kernels.w4a16 import kernel_name
    assert kernel_name(M, N, K).startswith("w4a16_mfma_x_kernel<")
    _run(M, N, K)


def test_mfma_x_bias_strided_rows_and_repeat():
    from kernels.w4a16 import kernel_name
    assert kernel_name(7, 2048, 1536).startswith("w4a16_mfma_x_kernel<")
    _run(7, 2048, 1536, bias=True)
    x, qw, s, z, _ = _make(7, 2048, 1536, 5)
    big = torch.zeros(7, 2048, dtype=torch.float16, device="cuda")
    big[:, :1536] = dev(x)
    qwd, sd, zd = dev(qw), dev(s), dev(z)
    a = w4a16_matmul(big[:, :1536], qwd, sd, zd)
    assert_north_star(a, w4a16_ref(x, qw, s, z))
    b = w4a16_matmul(big[:, :1536], qwd, sd, zd)
    assert torch.equal(a, b)  # deterministic


@pytest.mark.parametrize("M", [16, 5])
def test_mfma_x_one_hot_rows_reproduce_dequantized_weight(M):
    """Row m = e_k(m): every output row is a column of dequant(W) exactly, for every k of K = 1536
    (even and odd nibbles, all twelve groups, every packed row of the LDS records)."""
    from kernels.w4a16 import kernel_name
    N, K = 1024, 1536
    assert kernel_name(M, N, K).startswith("w4a16_mfma_x_kernel<")
    _, qw, s, z, _ = _make(1, N, K, 11)
    deq = dequantize_ref(qw, s, z, 128)
    qwd, sd, zd = dev(qw), dev(s), dev(z)
    rng = np.random.default_rng(3)
    order = rng.permutation(K)
    for c in range(0, K, M):
        ks = order[c:c + M]
        x = torch.zeros(len(ks), K, dtype=torch.float16, device="cuda")
        x[torch.arange(len(ks)), torch.as_tensor(ks)] = 1.0
        got = w4a16_matmul(x, qwd, sd, zd).cpu().numpy()
        assert np.array_equal(bits16(got), bits16(np.ascontiguousarray(deq[:, ks].T))), c


@pytest.mark.parametrize("M", [16, 6])
def test_mfma_x_64_column_tiles_one_hot(M):
    """64-column tiles (wide shapes from 5 rows: each lane's four words per packed row feed four
    MFMA tiles): one-hot rows return columns of dequant(W) exactly over K = 1536, N = 16384."""
    from kernels.w4a16 import kernel_name
    N, K = 16384, 1536
    assert kernel_name(M, N, K).endswith(", 4, false>")
    _, qw, s, z, _ = _make(1, N, K, 12)
    deq = dequantize_ref(qw, s, z, 128)
    qwd, sd, zd = dev(qw), dev(s), dev(z)
    order = np.random.default_rng(4).permutation(K)
    for c in range(0, K, 4 * M):  # a quarter of K's positions, all twelve groups
        ks = order[c:c + M]
        x = torch.zeros(len(ks), K, dtype=torch.float16, device="cuda")
        x[torch.arange(len(ks)), torch.as_tensor(ks)] = 1.0
        got = w4a16_matmul(x, qwd, sd, zd).cpu().numpy()
        assert np.array_equal(bits16(got), bits16(np.ascontiguousarray(deq[:, ks].T))), c


@pytest.mark.parametrize("M", [16, 6])
def test_mfma_x_80_column_tiles_one_hot(M):
    """80-column tiles (64-column tiles would need more than 256 workgroups: gate_up's 17920
    columns run 224): four words per lane and packed row feed four MFMA tiles and a fifth word
    the fifth tile (column 64 + c16). One-hot rows return columns of dequant(W) exactly."""
    from kernels.w4a16 import config_for, kernel_name
    N, K = 17920, 1536
    assert kernel_name(M, N, K).endswith(", 4, true>") and "block_n=80" in config_for(M, N, K)
    _, qw, s, z, _ = _make(1, N, K, 13)
    deq = dequantize_ref(qw, s, z, 128)
    qwd, sd, zd = dev(qw), dev(s), dev(z)
    order = np.random.default_rng(5).permutation(K)
    for c in range(0, K, 4 * M):  # a quarter of K's positions, all twelve groups
        ks = order[c:c + M]
        x = torch.zeros(len(ks), K, dtype=torch.float16, device="cuda")
        x[torch.arange(len(ks)), torch.as_tensor(ks)] = 1.0
        got = w4a16_matmul(x, qwd, sd, zd).cpu().numpy()
        assert np.array_equal(bits16(got), bits16(np.ascontiguousarray(deq[:, ks].T))), c


@pytest.mark.parametrize("M", [5, 9, 16])
@pytest.mark.parametrize("N", [16900, 16960, 20480])
def test_mfma_x_80_column_tiles_tails(M, N):
    """80-column tiles with a partial last tile (16900: 20 columns, so the fifth tile's lanes and
    three quarters of the four-column lanes clamp; 16960: 16 columns) and the widest grid they
    take (20480: 256 tiles), with bias."""
    from kernels.w4a16 import kernel_name
    assert kernel_name(M, N, 1536).endswith(", 4, true>")
    _run(M, N, 1536, bias=True)


# ---------------------------------------------------------------- config 0 and config 2
def test_config0_headline():
    """Config 0: M=1, gate_up 17920 x 1536, seed 0 (weights quantized by the oracle)."""
    e = _run(1, 17920, 1536, seed=0)
    assert e["rel_l2"] < 1e-3


@pytest.mark.parametrize("M", [1, 2, 4, 16])
@pytest.mark.parametrize("name,N,K", cases.QWEN_LINEARS)
def test_config2_qwen_shapes(name, N, K, M):
    _run(M, N, K, seed=2)


def test_qkv_fused_with_bias():
    """The e2e qkv projection: 2048 x 1536 with bias (decode key (1, 2048, 1536, True))."""
    _run(1, 2048, 1536, bias=True)


# ---------------------------------------------------------------- the native decode entry
@pytest.mark.parametrize("M", [1, 2, 3, 4, 7, 8, 16])
@pytest.mark.parametrize("split", [None, 1, 3, 4])
def test_decode_entry(M, split):
    """The reference's cases (tests/test_w4a16_cuda.py:23-27) with its explicit splits 1 and 4,
    a three-way split, and the library's table."""
    x, qw, s, z, _ = _make(M, 1536, 1536, 2)
    out = w4a16_decode_cuda(dev(x), dev(qw), dev(s), dev(z), split_k=split)
    assert out.shape == (M, 1536) and out.dtype == torch.float16
    assert_north_star(out, w4a16_ref(x, qw, s, z))


@pytest.mark.parametrize("N,K", [(2048, 1536), (17920, 1536), (1536, 8960), (4096, 14336)])
def test_decode_entry_autosplit(N, K):
    """tests/test_w4a16_cuda.py:30-33: one and 16 rows on the library's split table."""
    _run(1, N, K, entry=w4a16_decode_cuda)
    _run(16, N, K, entry=w4a16_decode_cuda)


def test_decode_entry_odd_n_split_bias_and_rows():
    """tests/test_w4a16_cuda.py:36-45: N = 1000 split 3 with bias, N = 132, and 17 rows refused."""
    for M, N, K, split in ((5, 1000, 1024, 3), (1, 132, 256, 1)):
        x, qw, s, z, b = _make(M, N, K, 5, bias=True)
        out = w4a16_decode_cuda(dev(x), dev(qw), dev(s), dev(z), bias=dev(b), split_k=split)
        assert_north_star(out, w4a16_ref(x, qw, s, z, 128, b))
    x, qw, s, z, _ = _make(17, 128, 128, 5)
    with pytest.raises(RuntimeError):
        w4a16_decode_cuda(dev(x), dev(qw), dev(s), dev(z), split_k=1)


# ------------------------------------------- the reference's config keys (tests/test_w4a16.py)
REF_CFG = dict(BLOCK_M=16, BLOCK_N=32, BLOCK_K=64, SPLIT_K=1, GROUP_M=8)
REF_GEMV = dict(GEMV=True, BLOCK_N=32, BLOCK_K=64, SPLIT_K=1)


@pytest.mark.parametrize("M,N,K", [(1, 64, 256), (3, 40, 128), (17, 96, 384)])
def test_reference_direct_small(M, N, K):
    _run(M, N, K, config=REF_CFG)


@pytest.mark.parametrize("split", [2, 3])
def test_reference_split_k_small(split):
    """SPLIT_K is honoured: K = 512 is 4 groups of 128, dealt evenly over 2 or 3 workgroups."""
    cfg = {**REF_CFG, "SPLIT_K": split}
    assert config_for(2, 48, 512, 128, cfg) == f"valu,block_n=32,split_k={split},factored"
    _run(2, 48, 512, config=cfg)


def test_reference_bias_both_paths():
    _run(1, 64, 256, bias=True, config=REF_CFG)
    _run(1, 64, 256, bias=True, config={**REF_CFG, "SPLIT_K": 2})


@pytest.mark.parametrize("N,K", [(64, 256), (40, 384), (96, 128)])
@pytest.mark.parametrize("split", [1, 3])
def test_reference_gemv(N, K, split):
    _run(1, N, K, config={**REF_GEMV, "SPLIT_K": split})


@pytest.mark.parametrize("split", [1, 2])
def test_reference_gemv_factored(split):
    _run(1, 96, 384, config={**REF_GEMV, "SPLIT_K": split, "FACTORED": True})
    _run(1, 64, 256, bias=True, config={**REF_GEMV, "FACTORED": True, "BLOCK_K": 128})


def test_reference_gemv_bias_and_block_k_128():
    _run(1, 64, 256, bias=True, config=REF_GEMV)
    _run(1, 64, 256, bias=True, config={**REF_GEMV, "SPLIT_K": 2, "BLOCK_K": 128})
    _run(5, 64, 256, config={**REF_CFG, "BLOCK_K": 128, "BLOCK_N": 64})


@pytest.mark.parametrize("M", [1, 2, 4, 8, 16])
def test_reference_decode_shape_8960x1536(M):
    """The reference's extra decode shape (tests/test_w4a16.py:84: N = 8960, K = 1536)."""
    _run(M, 8960, 1536)


@pytest.mark.parametrize("M", [33, 128, 2048])
def test_reference_prefill_8960x1536(M):
    """tests/test_w4a16.py:89-97: the (8960, 1536) prefill shape at the reference's rows."""
    _run(M, 8960, 1536)


# ------------------------------------------------------------- prefill rows (M > 16)
@pytest.mark.parametrize("M", [17, 32, 33, 65, 100, 128, 256])
@pytest.mark.parametrize("N,K,bias", [(2048, 1536, True), (17920, 1536, False),
                                      (1536, 8960, False), (96, 384, True)])
@pytest.mark.parametrize("path", ["blocks", "gemm"])
def test_prefill_native_rows(M, N, K, bias, path):
    """Prefill rows (the reference's prefill path, w4a16.py:264-268 and tests/test_w4a16.py:93-97)
    through the MFMA kernel in 16- or 32-row blocks and through the prefill GEMM: row tails inside a
    tile, bias, every Qwen width class."""
    _run(M, N, K, bias=bias, config={"prefill": path})


@pytest.mark.parametrize("M", [300, 512, 2048])
@pytest.mark.parametrize("N,K", [(2048, 1536), (1536, 1536), (17920, 1536), (1536, 8960)])
def test_prefill_gemm_reference_sizes(M, N, K):
    """The library's choice for many rows (the prefill GEMM) at the reference's slow-test size
    (M = 2048, tests/test_w4a16.py:93-97) on every Qwen2.5-1.5B linear shape, and row tails."""
    _run(M, N, K, bias=(N == 2048))


@pytest.mark.parametrize("gs", [64, 128, 256])
def test_prefill_gemm_group_sizes(gs):
    _run(200, 4096, 2048, gs=gs, config={"prefill": "gemm"})
    _run(130, 17920, 1024, gs=gs, config={"prefill": "gemm"})


def test_prefill_group_32_takes_the_blocks():
    """The GEMM steps K by 64; group 32 keeps the row blocks, still correct."""
    _run(200, 1024, 512, gs=32)


def test_prefill_gemm_strided_rows_and_narrow_n():
    x, qw, s, z, _ = _make(150, 96, 768, 21)
    wide = np.zeros((150, 1024), dtype=np.float16)
    wide[:, 100:868] = x
    xs = dev(wide)[:, 100:868]
    assert xs.stride(0) == 1024
    out = w4a16_matmul(xs, dev(qw), dev(s), dev(z), config={"prefill": "gemm"})
    assert_north_star(out, w4a16_ref(x, qw, s, z))


def test_prefill_gemm_32_row_tiles_with_tail():
    """qkv-like short K at about 500 rows runs 32-row tiles on two column groups and two K
    groups; 500 rows leave a partial last row tile."""
    _run(500, 2048, 1536, bias=True, config={"prefill": "gemm"})
    _run(512, 1536, 1536, config={"prefill": "gemm"})


def test_prefill_gemm_long_k_row_tiles_fast_with_tail():
    """Long K with 16 row tiles puts the row tiles on the grid's fast axis; 2000 rows leave a
    partial last row tile, with the K split and its reduce launch."""
    _run(2000, 1536, 8960, bias=True, config={"prefill": "gemm"})


def test_prefill_gemm_two_k_groups_odd_steps():
    """Two K groups in a workgroup over 33 K-steps of 64 (17 and 16: the second group takes one
    barrier-only step), a partial last column tile (N = 1000), row tails, on one and two column
    groups (M = 300 and 2048)."""
    _run(300, 1000, 2112, gs=64, config={"prefill": "gemm"})
    _run(2048, 1000, 2112, gs=64, bias=True, config={"prefill": "gemm"})


def test_prefill_gemm_one_hot_rows_reproduce_dequantized_weight():
    """x = e_k rows through the GEMM: row m of the output is column k of dequant(W) bit for bit,
    so each weight is dequantized exactly as dequantize_ref does it."""
    N, K = 17920, 1536
    _, qw, s, z, _ = _make(1, N, K, 6)
    ks = [0, 7, 64, 130, 511, 1024, 1535, 1000, 5] * 15  # 135 rows: two row tiles, a tail
    x = np.zeros((len(ks), K), dtype=np.float16)
    x[np.arange(len(ks)), ks] = 1.0
    out = w4a16_matmul(dev(x), dev(qw), dev(s), dev(z), config={"prefill": "gemm"})
    deq = dequantize_ref(qw, s, z)
    assert np.array_equal(bits16(out), bits16(deq[:, ks].T))


@pytest.mark.parametrize("gs", [32, 64, 256])
def test_prefill_native_group_sizes(gs):
    _run(48, 4096, 2048, gs=gs, config={"prefill": "blocks"})
    _run(40, 17920, 1024, gs=gs, config={"prefill": "blocks"})


def test_prefill_paths_agree():
    """The prefill paths (GEMM, row blocks, the library's choice) meet the bar on the same
    inputs, and an unknown path name is rejected."""
    for path in ("gemm", "blocks", "native"):
        _run(300, 2048, 1536, config={"prefill": path})
    with pytest.raises(ValueError, match="prefill"):
        _run(300, 2048, 1536, config={"prefill": "dequant"})


@pytest.mark.parametrize("block_n,split_k", [(128, 0), (256, 0), (0, 3), (256, 5)])
def test_prefill_gemm_tile_and_split_arguments(block_n, split_k):
    """block_n and split_k pick the GEMM's tile and K split when the GEMM is forced."""
    _run(300, 1536, 8960, config={"prefill": "gemm", "block_n": block_n, "split_k": split_k})
    _run(130, 2048, 1536, bias=True, config={"prefill": "gemm", "block_n": block_n, "split_k": split_k})


def test_prefill_one_hot_rows_reproduce_dequantized_weight():
    """x = e_k rows (k = 0, 7, 130, ...): row m of the output is column k of dequant(W), exact."""
    N, K = 17920, 1536
    _, qw, s, z, _ = _make(1, N, K, 5)
    ks = [0, 7, 130, 511, 1024, 1535] * 6  # 36 rows, two row blocks
    x = np.zeros((len(ks), K), dtype=np.float16)
    x[np.arange(len(ks)), ks] = 1.0
    out = w4a16_matmul(dev(x), dev(qw), dev(s), dev(z), config={"prefill": "blocks"})
    deq = dequantize_ref(qw, s, z)
    assert np.array_equal(bits16(out), bits16(deq[:, ks].T))


def test_decode_entry_rejects_17_rows():
    """As the reference's CUDA entry (tests/test_w4a16_cuda.py:43-45)."""
    with pytest.raises(RuntimeError):
        _run(17, 128, 128, entry=w4a16_decode_cuda)


def test_deterministic():
    x, qw, s, z, _ = _make(1, 17920, 1536, 0)
    a = w4a16_matmul(dev(x), dev(qw), dev(s), dev(z))
    b = w4a16_matmul(dev(x), dev(qw), dev(s), dev(z))
    assert torch.equal(a, b)


def test_prefill_gemm_k_split_deterministic_and_leaves_workspace_clean():
    """Long K and few tiles (down at 512 rows) split K over workgroups; the partials are summed
    in split order by a second launch (same bits every call), and zeroed, so a decode split-K
    call right after sees a clean workspace."""
    x, qw, s, z, _ = _make(512, 1536, 8960, 22)
    args = (dev(x), dev(qw), dev(s), dev(z))
    outs = [w4a16_matmul(*args, config={"prefill": "gemm"}) for _ in range(3)]
    assert all(torch.equal(o, outs[0]) for o in outs[1:])
    assert_north_star(outs[0], w4a16_ref(x, qw, s, z))
    x1 = x[:1].copy()
    y1 = w4a16_matmul(dev(x1), *args[1:], config={"split_k": 5})
    assert_north_star(y1, w4a16_ref(x1, qw, s, z))


def test_choice_export_records_only_the_library_choice():
    """A call whose config forces a variant records nothing; a call left to the library records
    the table's choice for its decode key, which export/import round-trip (w4a16.py:322-342)."""
    from kernels import w4a16 as mod

    mod._decode_choice.clear()
    x, qw, s, z, _ = _make(1, 1536, 1536, 3)
    args = (dev(x), dev(qw), dev(s), dev(z))
    w4a16_matmul(*args, config={"GEMV": True, "block_n": 32})
    assert mod.export_choices() == {}
    w4a16_matmul(*args)
    exported = mod.export_choices()
    assert exported == {"1,1536,1536,False": mod.config_for(1, 1536, 1536)}
    mod._decode_choice.clear()
    mod.import_choices(exported)
    assert mod.export_choices() == exported


@pytest.mark.parametrize("M", [17, 33, 65, 100, 128])
@pytest.mark.parametrize("split", [None, 2, 3, 8])
def test_prefill_blocks_split_k(M, split):
    """Prefill rows of a long-K shape on the MFMA row blocks with K split over workgroups
    (the library's choice below about 200 rows on down: 16-row blocks in 5 / 3 / 2 splits at
    17 / 33 / 65 rows, 32-row blocks in 2 at 100 and 128; explicit splits run 32-row blocks): each row block's
    split tiles meet in their own fixed-point words, the last row block ragged. Repeated calls
    give the same bits (every word is back to zero after a call)."""
    cfg = {"prefill": "blocks"} if split is None else {"prefill": "blocks", "split_k": split}
    _run(M, 1536, 8960, bias=True, config=cfg)
    x, qw, s, z, b = _make(M, 1536, 8960, 9, bias=True)
    args = (dev(x), dev(qw), dev(s), dev(z))
    y0 = w4a16_matmul(*args, bias=dev(b), config=cfg)
    y1 = w4a16_matmul(*args, bias=dev(b), config=cfg)
    assert torch.equal(y0, y1)


# ---------------------------------------------------- prefill rows on 16- and 32-row blocks (plan)
@pytest.mark.parametrize("M", [17, 40, 65, 100, 144, 160, 192])
@pytest.mark.parametrize("N,K", [(1536, 1536), (2048, 1536), (1536, 8960), (1000, 1536), (2064, 512)])
def test_prefill_row_blocks_default_plan(M, N, K):
    """The library's choice at prefill rows: 16-row blocks where they fit in 256 workgroups (short
    K whole, long K in 2-5 splits), 32-row blocks in K splits up to 256 workgroups (128-column
    tiles in 3 splits for down at 192 rows), the prefill GEMM past that; ragged last row block, a
    partial last column tile (N = 1000, 2064)."""
    _run(M, N, K, bias=(N == 2048))


@pytest.mark.parametrize("N,K", [(1536, 8960), (2048, 1536)])
def test_prefill_16_row_blocks_one_hot_rows_exact(N, K):
    """x = e_k rows through the 16-row blocks (M = 40: three blocks, the last ragged; down in
    three K splits, qkv whole): row m of the output is column k of dequant(W) bit for bit."""
    M = 40
    assert kernel_name(M, N, K).split(", ")[3] == "1"
    _, qw, s, z, _ = _make(1, N, K, 7)
    ks = [(m * 211) % K for m in range(M)]
    x = np.zeros((M, K), dtype=np.float16)
    x[np.arange(M), ks] = 1.0
    out = w4a16_matmul(dev(x), dev(qw), dev(s), dev(z))
    deq = dequantize_ref(qw, s, z)
    assert np.array_equal(bits16(out), bits16(deq[:, ks].T))
