"""The reference's Triton config keys (SPLIT_K, BLOCK_N) as this build reads them, checked through
the library's plan query (ldk_w4a16_config / ldk_w8a16_config, host code only: no GPU needed).
The reference's tests force splits and tile widths with these keys (tests/test_w4a16.py:33-66,
tests/test_fp8.py:37-48); here a forced SPLIT_K must run that many workgroups along K, and a
BLOCK_N must become the tile width where the kernel the call runs takes it."""

import pytest

from kernels import fp8, w4a16

CFG = dict(BLOCK_M=16, BLOCK_N=32, BLOCK_K=64, SPLIT_K=1, GROUP_M=8)
GEMV = dict(GEMV=True, BLOCK_N=32, BLOCK_K=64, SPLIT_K=1)
FP8_CFG = dict(BLOCK_M=16, BLOCK_N=32, BLOCK_K=32, SPLIT_K=1, GROUP_M=8)


def _fields(desc: str) -> dict:
    return dict(kv.split("=") for kv in desc.split(",") if "=" in kv)


@pytest.mark.parametrize("split", [1, 2, 3, 4])
def test_w4a16_split_k_runs_that_many_splits(split):
    """K = 512 at group 128 is 4 groups: 3 splits deal them 2 + 1 + 1 (the reference's
    test_split_k_small, tests/test_w4a16.py:41-44)."""
    f = _fields(w4a16.config_for(2, 48, 512, 128, {**CFG, "SPLIT_K": split}))
    assert int(f["split_k"]) == split


def test_w4a16_split_k_at_most_the_groups():
    """A split is a range of quantization groups: K = 256 (2 groups) takes at most 2."""
    assert _fields(w4a16.config_for(1, 64, 256, 128, {**GEMV, "SPLIT_K": 3}))["split_k"] == "2"
    assert _fields(w4a16.config_for(1, 96, 128, 128, {**GEMV, "SPLIT_K": 3}))["split_k"] == "1"
    assert _fields(w4a16.config_for(1, 40, 384, 128, {**GEMV, "SPLIT_K": 3}))["split_k"] == "3"


def test_w4a16_lowercase_keys_win():
    f = _fields(w4a16.config_for(1, 1536, 1536, 128, {**CFG, "split_k": 4, "block_n": 16}))
    assert f["split_k"] == "4" and f["block_n"] == "16"


@pytest.mark.parametrize("M,N,K,bn", [(1, 64, 256, 32), (3, 40, 128, 32), (5, 64, 256, 64),
                                      (16, 1536, 1536, 32), (17, 96, 384, 32)])
def test_w4a16_block_n_taken_where_the_kernel_has_it(M, N, K, bn):
    f = _fields(w4a16.config_for(M, N, K, 128, {**CFG, "BLOCK_N": bn}))
    assert int(f["block_n"]) == bn


def test_w4a16_block_n_ignored_where_the_kernel_lacks_it():
    """The VALU kernels stop at 64 columns: BLOCK_N = 128 with GEMV keeps the table's width, where
    an explicit block_n = 128 is refused as the call would refuse it."""
    table = _fields(w4a16.config_for(1, 1536, 1536, 128, {"GEMV": True}))
    f = _fields(w4a16.config_for(1, 1536, 1536, 128, {**GEMV, "BLOCK_N": 128}))
    assert f["block_n"] == table["block_n"]
    with pytest.raises(RuntimeError):
        w4a16.config_for(1, 1536, 1536, 128, {"GEMV": True, "block_n": 128})


def test_w4a16_table_choices_unchanged_by_the_query():
    assert w4a16.config_for(1, 17920, 1536) == w4a16.config_for(1, 17920, 1536, 128, {})
    assert w4a16.config_for(2048, 17920, 1536).startswith("gemm,")
    assert w4a16.config_for(16, 1536, 8960).startswith("mfma,")


@pytest.mark.parametrize("M,N,K", [(1, 64, 128), (5, 40, 96), (17, 96, 256)])
def test_fp8_reference_direct_cases_plan(M, N, K):
    f = _fields(fp8.config_for(M, N, K, FP8_CFG))
    assert f["split_k"] == "1"


def test_fp8_split_and_gemv_keys():
    assert _fields(fp8.config_for(2, 48, 256, {**FP8_CFG, "SPLIT_K": 3}))["split_k"] == "3"
    gemv = {"GEMV": True, "BLOCK_N": 32, "BLOCK_K": 64, "SPLIT_K": 2}
    assert fp8.config_for(1, 48, 256, gemv) == "valu,block_n=32,split_k=2"


def test_fp8_column_tails_plan():
    """N % 16 != 0: 64-column MFMA tiles where N % 8 != 0, 128-column VALU tiles, no prefill GEMM."""
    assert fp8.config_for(5, 44, 96).startswith("mfma,block_n=64")
    assert fp8.config_for(1, 44, 96).startswith("valu,block_n=128")
    assert fp8.config_for(512, 1000, 1536).startswith("mfma,")
    assert fp8.config_for(512, 1024, 1536).startswith("gemm,")
    with pytest.raises(RuntimeError):
        fp8.config_for(1, 42, 96)
    with pytest.raises(RuntimeError):
        fp8.config_for(5, 44, 96, {"MFMA": True, "block_n": 128})


def test_fp8_prefill_tiles_of_the_wide_shapes():
    """The e4m3 prefill GEMM's tile on gate_up (17920 x 1536): 4 x 64 columns in one K group from
    256 rows (its 4-wave two-group tiles do not fit the LDS), 2 x 64 columns below."""
    assert fp8.config_for(128, 17920, 1536) == "gemm,block_n=128,split_k=1"
    for M in (256, 384, 512, 2048):
        assert fp8.config_for(M, 17920, 1536) == "gemm,block_n=256,split_k=1"


def test_w4a16_prefill_tiles_of_the_wide_shapes():
    """The int4 prefill GEMM's tile on gate_up: 4 x 64 columns in two K groups unless that gives
    257-383 tiles (256 and 320 rows), where 2 x 64 columns spread twice the workgroups evenly."""
    cfg = {"prefill": "gemm"}
    for M, bn in ((128, 128), (192, 256), (256, 128), (320, 128), (384, 256), (512, 256)):
        assert w4a16.config_for(M, 17920, 1536, 128, cfg) == f"gemm,block_n={bn},split_k=1", M


def test_w4a16_prefill_choice_of_the_narrow_shapes():
    """int4 narrow shapes keep the 32-row blocks up to 256 rows, and up to 511 rows while the
    blocks fit in 256 workgroups (64-column tiles x 32-row blocks); past that the prefill GEMM."""
    cases = (
        (256, 2048, 1536, "mfma"),   # qkv: 32 x 8 blocks
        (288, 2048, 1536, "gemm"),   # qkv: 32 x 9
        (288, 1536, 1536, "mfma"),   # o: 24 x 9
        (320, 1536, 8960, "mfma"),   # down: 24 x 10
        (352, 1536, 8960, "gemm"),   # down: 24 x 11
        (512, 256, 1536, "gemm"),    # 4 x 16, but 512 rows
        (64, 1536, 8960, "mfma"),
        (32, 17920, 1536, "gemm"),   # wide from 32 rows
        (31, 17920, 1536, "mfma"),
    )
    for M, N, K, path in cases:
        assert w4a16.config_for(M, N, K).startswith(path + ","), (M, N, K, w4a16.config_for(M, N, K))


def test_w4a16_prefill_row_blocks():
    """Prefill rows on the MFMA blocks: 16-row blocks (MT = 1, the fourth template argument)
    wherever they fit in 256 workgroups on short K; on long K where they split K at least twice
    over 192 or more workgroups, else 32-row blocks (MT = 2) with K split toward 256 workgroups,
    never past it, on 128-column tiles where those split into a grid half again as large."""
    cases = (  # M, N, K, MT, split_k
        (17, 2048, 1536, 1, 1), (128, 2048, 1536, 1, 1), (144, 2048, 1536, 2, 1),
        (160, 1536, 1536, 1, 1), (176, 1536, 1536, 2, 1),
        (17, 1536, 8960, 1, 5), (48, 1536, 8960, 1, 3), (80, 1536, 8960, 1, 2),
        (96, 1536, 8960, 2, 3), (128, 1536, 8960, 2, 2), (160, 1536, 8960, 2, 2),
        (192, 1536, 8960, 2, 3), (256, 1536, 8960, 2, 1), (20, 17920, 1536, 2, 1),
    )
    for M, N, K, mt, sk in cases:
        name = w4a16.kernel_name(M, N, K)
        assert name.startswith("w4a16_mfma_kernel<") and name.split(", ")[3] == str(mt), (M, N, K, name)
        assert _fields(w4a16.config_for(M, N, K))["split_k"] == str(sk), (M, N, K)
    assert w4a16.config_for(192, 1536, 8960).startswith("mfma,block_n=128,split_k=3")
    assert w4a16.config_for(192, 1536, 8960, 256).startswith("mfma,block_n=64,")  # group 256: 64 columns


def test_fp8_prefill_row_blocks():
    """e4m3 prefill rows: the 16-row blocks on narrow shapes while they fit in 256 workgroups,
    short K on 64-column tiles with K split toward 256 workgroups, long K (128-column tiles) while
    it still splits at least twice; the prefill GEMM past that and from 17 rows on wide shapes."""
    cases = (  # M, N, K, expected
        (17, 2048, 1536, "mfma,block_n=64,split_k=4"), (64, 2048, 1536, "mfma,block_n=64,split_k=2"),
        (128, 2048, 1536, "mfma,block_n=64,split_k=1"), (160, 2048, 1536, "gemm,"),
        (17, 1536, 1536, "mfma,block_n=64,split_k=5"), (160, 1536, 1536, "mfma,block_n=64,split_k=1"),
        (176, 1536, 1536, "gemm,"), (64, 1536, 8960, "mfma,block_n=128,split_k=5"),
        (128, 1536, 8960, "mfma,block_n=128,split_k=2"), (176, 1536, 8960, "gemm,"),
        (17, 17920, 1536, "gemm,"),
    )
    for M, N, K, want in cases:
        assert fp8.config_for(M, N, K).startswith(want), (M, N, K, fp8.config_for(M, N, K))
