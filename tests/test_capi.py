"""The C-ABI library (libldk_amd.so) on the CPU: it loads, exports every entry point declared in
include/ldk.h, shares torch's HIP runtime, and rejects bad arguments with status codes before
launching anything (no GPU is touched by these tests)."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from kernels import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "ldk.h"


def _declared() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(ldk_\w+)\s*\(", text, flags=re.M))


def test_header_declares_what_the_binding_binds():
    assert _declared() == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name


def test_abi_version_matches_header():
    m = re.search(r"#define LDK_ABI_VERSION (\d+)", HEADER.read_text())
    assert _lib.load().ldk_abi_version() == int(m.group(1))


def test_one_hip_runtime_per_process():
    """The library binds the libamdhip64 that torch loaded (one runtime, shared streams)."""
    _lib.load()
    maps = Path("/proc/self/maps").read_text().splitlines()
    hip = {line.split()[-1] for line in maps if "libamdhip64" in line}
    assert len(hip) == 1, hip


def _err(st):
    return st, _lib.load().ldk_last_error().decode()


def test_null_pointer_rejected():
    lib = _lib.load()
    st, msg = _err(lib.ldk_w4a16_matmul(None, 1536, None, None, None, None, None, 17920, 1, 17920,
                                        1536, 128, 0, 0, 0, None, 0, None))
    assert st == _lib.ERR_INVALID and "null" in msg


def test_decode_rejects_more_than_16_rows():
    """Reference: w4a16_decode_cuda raises for M = 17 (tests/test_w4a16_cuda.py:43-45)."""
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    st, msg = _err(lib.ldk_w4a16_decode(p, 128, p, p, p, None, p, 128, 17, 128, 128, 128, 0, None, 0,
                                        None))
    assert st == _lib.ERR_UNSUPPORTED and "16" in msg


@pytest.mark.parametrize("K,gs", [(1536, 96), (1536, 4), (1000, 128)])
def test_bad_group_size_rejected(K, gs):
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    st, _ = _err(lib.ldk_w4a16_matmul(p, K, p, p, p, None, p, 64, 1, 64, K, gs, 0, 0, 0, None, 0,
                                      None))
    assert st == _lib.ERR_INVALID


def test_split_without_workspace_rejected():
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    st, msg = _err(lib.ldk_w4a16_matmul(p, 1536, p, p, p, None, p, 1536, 1, 1536, 1536, 128, 0, 4,
                                        0, None, 0, None))
    assert st == _lib.ERR_INVALID and "workspace" in msg


def test_misaligned_pointer_rejected():
    lib = _lib.load()
    p, bad = ctypes.c_void_p(256), ctypes.c_void_p(258)
    st, _ = _err(lib.ldk_w4a16_matmul(bad, 256, p, p, p, None, p, 64, 1, 64, 256, 128, 0, 0, 0, None,
                                      0, None))
    assert st == _lib.ERR_ALIGN


def test_factored_valu_takes_two_rows():
    """The factored VALU kernel takes M <= 2; more rows run the factored form on the MFMA kernel,
    so FACTORED with the VALU path is refused from 3 rows (before any launch)."""
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    st, msg = _err(lib.ldk_w4a16_matmul(p, 256, p, p, p, None, p, 64, 3, 64, 256, 128, 0, 0,
                                        _lib.FACTORED | _lib.PATH_VALU, None, 0, None))
    assert st == _lib.ERR_UNSUPPORTED and "M <= 2" in msg


def test_exact_is_not_the_mfma_kernel():
    """The MFMA kernel computes the factored form: EXACT with the MFMA path is refused."""
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    st, msg = _err(lib.ldk_w4a16_matmul(p, 256, p, p, p, None, p, 64, 16, 64, 256, 128, 0, 0,
                                        _lib.EXACT | _lib.PATH_MFMA, None, 0, None))
    assert st == _lib.ERR_UNSUPPORTED and "factored" in msg


def test_w8a16_swiglu_validates_before_launch():
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    st, msg = _err(lib.ldk_w8a16_swiglu_matmul(p, p, p, None, p, 42, 256, None, 0, None))
    assert st == _lib.ERR_UNSUPPORTED and "multiple of 4" in msg
    st, _ = _err(lib.ldk_w8a16_swiglu_matmul(p, p, p, None, p, 64, 100, None, 0, None))
    assert st == _lib.ERR_UNSUPPORTED
    st, _ = _err(lib.ldk_w8a16_swiglu_matmul(p, ctypes.c_void_p(264), p, None, p, 64, 256, None, 0, None))
    assert st == _lib.ERR_ALIGN


def test_w8a16_rmsnorm_validates_before_launch():
    lib = _lib.load()
    p, q = ctypes.c_void_p(256), ctypes.c_void_p(512)
    st, msg = _err(lib.ldk_w8a16_rmsnorm_matmul(p, q, q, p, 1e-6, p, p, None, p, 64, 256, None, 0,
                                                None))
    assert st == _lib.ERR_INVALID and "alias" in msg
    st, _ = _err(lib.ldk_w8a16_rmsnorm_matmul(p, q, None, p, 1e-6, p, p, None, p, 64, 256, None, 0,
                                              None))
    assert st == _lib.ERR_INVALID
    st, _ = _err(lib.ldk_w8a16_rmsnorm_matmul(ctypes.c_void_p(258), None, None, p, 1e-6, p, p, None,
                                              p, 64, 256, None, 0, None))
    assert st == _lib.ERR_ALIGN
    st, _ = _err(lib.ldk_w8a16_rmsnorm_matmul(p, None, None, p, 1e-6, p, p, None, p, 42, 256, None,
                                              0, None))
    assert st == _lib.ERR_UNSUPPORTED


def test_residual_stats_pair_validation():
    lib = _lib.load()
    p, q = ctypes.c_void_p(256), ctypes.c_void_p(4096)
    assert lib.ldk_w4a16_row_stats_count(1536, 1536, 128) == 96
    assert lib.ldk_w4a16_row_stats_count(1536, 1000, 128) < 0
    # h_out aliasing x
    st, msg = _err(lib.ldk_w4a16_matmul_residual_stats(p, q, p, q, p, p, p, None, 1536, 1536, 128,
                                                       None, 0, None))
    assert st == _lib.ERR_INVALID and "alias" in msg
    # more tiles than partials
    st, _ = _err(lib.ldk_w4a16_matmul_residual_stats(p, q, q, q, p, p, p, None, 16384, 1536, 128,
                                                     None, 0, None))
    assert st == _lib.ERR_UNSUPPORTED
    st, _ = _err(lib.ldk_w4a16_rmsnorm_stats_matmul(p, q, 0, p, 1e-6, p, p, p, None, p, 2048, 1536,
                                                    128, None, 0, None))
    assert st == _lib.ERR_UNSUPPORTED


def test_rmsnorm_residual_pairing_rejected():
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    st, _ = _err(lib.ldk_rmsnorm(p, 64, p, 64, p, p, 64, None, 64, 1, 64, 1e-6, None))
    assert st == _lib.ERR_INVALID


def test_fused_entries_validate_before_launch():
    lib = _lib.load()
    p, q = ctypes.c_void_p(256), ctypes.c_void_p(512)
    # residual_out aliasing the residual
    st, msg = _err(lib.ldk_w4a16_rmsnorm_matmul(p, q, q, p, 1e-6, p, p, p, None, p, 1536, 1536, 128,
                                                None, 0, None))
    assert st == _lib.ERR_INVALID and "alias" in msg
    # residual without residual_out
    st, _ = _err(lib.ldk_w4a16_rmsnorm_matmul(p, q, None, p, 1e-6, p, p, p, None, p, 1536, 1536,
                                              128, None, 0, None))
    assert st == _lib.ERR_INVALID
    # no norm weight
    st, _ = _err(lib.ldk_w4a16_rmsnorm_matmul(p, None, None, None, 1e-6, p, p, p, None, p, 1536,
                                              1536, 128, None, 0, None))
    assert st == _lib.ERR_INVALID
    # a group size the fused kernels are not built for (64) is reported, not launched
    st, msg = _err(lib.ldk_w4a16_swiglu_matmul(p, p, p, p, None, p, 1536, 1536, 64, None, 0, None))
    assert st == _lib.ERR_UNSUPPORTED and "128" in msg
    st, _ = _err(lib.ldk_w4a16_swiglu_matmul(None, p, p, p, None, p, 1536, 1536, 128, None, 0, None))
    assert st == _lib.ERR_INVALID


def test_attention_merge_entries_validate_before_launch():
    """The o projections that merge the decode attention's range partials in their x staging
    (int4 and e4m3) check the head geometry, the ranges and the pointers before they look for the
    partials or launch."""
    lib = _lib.load()
    p, q = ctypes.c_void_p(256), ctypes.c_void_p(4096)
    odd = ctypes.c_void_p(264)  # 8-byte but not 16-byte aligned

    def w8(pos=p, max_len=416, rlen=128, nq=12, wq=p, N=1536, K=1536, ws=None, ws_bytes=0):
        return _err(lib.ldk_w8a16_attn_matmul(pos, max_len, rlen, nq, wq, q, None, q, N, K, ws, ws_bytes, None))

    assert w8(pos=None)[0] == _lib.ERR_INVALID
    assert w8(nq=11)[0] == _lib.ERR_INVALID  # K != nq * 128
    assert w8(nq=0, K=0)[0] == _lib.ERR_INVALID
    st, msg = w8(rlen=48)  # not a multiple of 32
    assert st == _lib.ERR_UNSUPPORTED and "ranges" in msg
    assert w8(max_len=4096)[0] == _lib.ERR_UNSUPPORTED  # 32 ranges of 128: more than the merge holds
    assert w8(N=42)[0] == _lib.ERR_UNSUPPORTED
    assert w8(wq=odd)[0] == _lib.ERR_ALIGN
    assert w8(ws_bytes=1 << 20)[0] == _lib.ERR_ALIGN  # a workspace size without a workspace

    def w4(pos=p, max_len=416, rlen=128, nq=12, K=1536, gs=128, h_out=q):
        return _err(lib.ldk_w4a16_attn_matmul_residual_stats(pos, max_len, rlen, nq, p, h_out, q, p, p, p, None,
                                                             1536, K, gs, None, 0, None))

    assert w4(pos=None)[0] == _lib.ERR_INVALID
    assert w4(nq=11)[0] == _lib.ERR_INVALID
    assert w4(gs=64)[0] == _lib.ERR_UNSUPPORTED
    assert w4(rlen=48)[0] == _lib.ERR_UNSUPPORTED
    assert w4(max_len=1024)[0] == _lib.ERR_UNSUPPORTED  # 8 ranges of 128
    assert w4(h_out=ctypes.c_void_p(4100))[0] == _lib.ERR_ALIGN


def test_matmul_swiglu_plan_and_validation():
    """ldk_w4a16_matmul_swiglu runs where the library's plan is the prefill GEMM on paired column
    groups of 64-row tiles with no K split, and refuses other shapes and bad outputs before any
    launch."""
    lib = _lib.load()
    assert lib.ldk_w4a16_matmul_swiglu_applies(128, 17920, 1536, 128) == 1
    assert lib.ldk_w4a16_matmul_swiglu_applies(512, 17920, 1536, 128) == 1
    assert lib.ldk_w4a16_matmul_swiglu_applies(2048, 17920, 1536, 128) == 0  # 128-row tiles
    assert lib.ldk_w4a16_matmul_swiglu_applies(1, 17920, 1536, 128) == 0     # decode rows
    assert lib.ldk_w4a16_matmul_swiglu_applies(128, 1536, 8960, 128) == 0    # down: row blocks
    p = ctypes.c_void_p(256)

    def call(M=128, N=17920, out=p, ldo=8960):
        return _err(lib.ldk_w4a16_matmul_swiglu(p, 1536, p, p, p, None, out, ldo, M, N, 1536, 128, None, 0, None))

    assert call(ldo=4000)[0] == _lib.ERR_ALIGN       # ldo < N / 2
    assert call(ldo=8962)[0] == _lib.ERR_ALIGN       # ldo % 4
    assert call(out=ctypes.c_void_p(260))[0] == _lib.ERR_ALIGN
    st, msg = call(M=2048)
    assert st == _lib.ERR_UNSUPPORTED and "applies" in msg


def test_w8a16_matmul_swiglu_plan_and_validation():
    """The e4m3 twin: the GEMM on paired 4-wave column groups (gate_up from 200 to 512 rows),
    refused on 2-wave tiles (whose waves read half lines), the decode rows, the row blocks and
    bad outputs before any launch."""
    lib = _lib.load()
    assert lib.ldk_w8a16_matmul_swiglu_applies(256, 17920, 1536) == 1
    assert lib.ldk_w8a16_matmul_swiglu_applies(512, 17920, 1536) == 1
    assert lib.ldk_w8a16_matmul_swiglu_applies(128, 17920, 1536) == 0    # 2-wave tiles
    assert lib.ldk_w8a16_matmul_swiglu_applies(8, 17920, 1536) == 0      # decode rows
    assert lib.ldk_w8a16_matmul_swiglu_applies(256, 1536, 8960) == 0     # down
    p = ctypes.c_void_p(256)

    def call(M=256, N=17920, out=p, ldo=8960):
        return _err(lib.ldk_w8a16_matmul_swiglu(p, 1536, p, p, None, out, ldo, M, N, 1536, None, 0, None))

    assert call(ldo=4000)[0] == _lib.ERR_ALIGN
    assert call(out=ctypes.c_void_p(260))[0] == _lib.ERR_ALIGN
    assert call(N=17922)[0] == _lib.ERR_UNSUPPORTED  # N % 4
    st, msg = call(M=8)
    assert st == _lib.ERR_UNSUPPORTED and "applies" in msg


def test_w8a16_n_multiple_of_4():
    """The reference masks columns, so any N runs there (N = 40 in tests/test_fp8.py:40); here N
    must be a multiple of 4 (N = 40 plans, N = 42 is refused before any launch)."""
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    st, msg = _err(lib.ldk_w8a16_matmul(p, 64, p, p, None, p, 42, 1, 42, 64, 0, 0, 0, None, 0, None))
    assert st == _lib.ERR_UNSUPPORTED and "multiple of 4" in msg
    for M in (1, 5, 17, 100):
        bn, sk, fl = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()  # in: the library's choice
        st = lib.ldk_w8a16_config(M, 40, 96, ctypes.byref(bn), ctypes.byref(sk), ctypes.byref(fl))
        assert st == 0, (M, lib.ldk_last_error())


def _config(M, N, K, gs=128, block_n=0, split_k=0, flags=0):
    """ldk_w4a16_config's plan for a call with these tuning arguments (in/out parameters)."""
    bn, sk, fl = ctypes.c_int(block_n), ctypes.c_int(split_k), ctypes.c_int(flags)
    st = _lib.load().ldk_w4a16_config(M, N, K, gs, ctypes.byref(bn), ctypes.byref(sk), ctypes.byref(fl))
    return st, bn.value, sk.value, fl.value


def test_config_query():
    st, bn, sk, fl = _config(1, 17920, 1536)
    assert st == 0 and bn in (16, 32, 64) and sk >= 1
    assert fl & _lib.FACTORED and fl & _lib.PATH_VALU
    st, bn, sk, fl = _config(16, 17920, 1536)
    assert st == 0 and fl & _lib.PATH_MFMA and bn == 80  # x staged in LDS, 80-column tiles
    # two rows: the factored VALU kernel; from three rows the MFMA kernel, also on small shapes
    st, bn, sk, fl = _config(2, 17920, 1536)
    assert st == 0 and fl & _lib.FACTORED and fl & _lib.PATH_VALU and bn == 32
    st, bn, sk, fl = _config(3, 1536, 1536)
    assert st == 0 and fl & _lib.PATH_MFMA
    # the prefill GEMM for many rows, and a call's tuning arguments as inputs
    st, bn, sk, fl = _config(2048, 17920, 1536)
    assert st == 0 and fl == _lib.PATH_GEMM
    st, bn, sk, fl = _config(1, 1536, 1536, block_n=16, split_k=3)
    assert st == 0 and (bn, sk) == (16, 3)
    # a query returns the status the call would: block_n 128 is not a VALU width
    st, *_ = _config(1, 1536, 1536, block_n=128, flags=_lib.PATH_VALU)
    assert st == _lib.ERR_UNSUPPORTED


def test_decode_rows_plan_kernels():
    """Decode rows 3-16 with group size 128 and K <= 1536 run the MFMA kernel with x staged in LDS;
    longer K (down), other group sizes and forced variants keep the wide-tile MFMA kernel, which
    also takes two rows of down; one and two rows otherwise the factored VALU kernel; more than 16
    the MFMA blocks."""
    from kernels.w4a16 import kernel_name
    # 80-column tiles where 64 columns need more than 256 workgroups and 80 at most 256
    assert kernel_name(16, 17920, 1536) == "w4a16_mfma_x_kernel<16, 12, 1, 4, true>"
    assert kernel_name(8, 17920, 1536) == "w4a16_mfma_x_kernel<8, 12, 1, 4, true>"
    assert kernel_name(5, 17920, 1536) == "w4a16_mfma_x_kernel<8, 12, 1, 4, true>"
    assert kernel_name(16, 16400, 1536) == "w4a16_mfma_x_kernel<16, 12, 1, 4, true>"  # N % 64 != 0
    assert kernel_name(16, 16384, 1536) == "w4a16_mfma_x_kernel<16, 12, 1, 4, false>"  # 256 x 64
    assert kernel_name(16, 20484, 1536) == "w4a16_mfma_x_kernel<16, 12, 1, 2, false>"  # past 256 x 80
    assert kernel_name(4, 17920, 1536) == "w4a16_mfma_x_kernel<4, 6, 2, 2, false>"
    assert kernel_name(8, 1536, 1536) == "w4a16_mfma_x_kernel<8, 12, 1, 2, false>"
    assert kernel_name(3, 4096, 512) == "w4a16_mfma_x_kernel<4, 6, 1, 2, false>"
    assert kernel_name(16, 256, 1536) == "w4a16_mfma_x_kernel<16, 12, 1, 2, false>"
    assert kernel_name(16, 200, 1536) == "w4a16_mfma_x_kernel<16, 12, 1, 2, false>"
    assert kernel_name(16, 1536, 8960).startswith("w4a16_mfma_kernel<")
    # down: 64 columns in 10 K splits up to 12 rows, 32 columns in 5 from 13 (half the words)
    from kernels.w4a16 import config_for
    assert config_for(12, 1536, 8960) == "mfma,block_n=64,split_k=10,factored"
    assert config_for(13, 1536, 8960) == config_for(16, 1536, 8960) == "mfma,block_n=32,split_k=5,factored"
    assert kernel_name(8, 1536, 1536, 64).startswith("w4a16_mfma_kernel<")
    assert kernel_name(16, 17920, 1536, 64).startswith("w4a16_mfma_kernel<")
    assert kernel_name(2, 17920, 1536).startswith("w4a16_m1_kernel<")
    assert kernel_name(2, 1536, 8960).startswith("w4a16_mfma_kernel<")  # two rows, narrow > 2 MB
    assert kernel_name(2, 1536, 1536).startswith("w4a16_m1_kernel<")
    assert kernel_name(17, 17920, 1536).startswith("w4a16_mfma_kernel<")


def test_workspace_size():
    assert _lib.load().ldk_workspace_bytes() >= 1 << 20


def test_python_ops_refuse_cpu_tensors():
    """No CPU path: the product ops raise instead of computing on the host."""
    from kernels.quant import quantize_rtn
    from kernels.rmsnorm import rmsnorm
    from kernels.w4a16 import w4a16_matmul

    w = torch.randn(64, 128).half()
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        rmsnorm(torch.randn(2, 64).half(), torch.ones(64).half())
    qw = torch.zeros(16, 64, dtype=torch.int32)
    s = torch.ones(1, 64).half()
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        w4a16_matmul(torch.randn(1, 128).half(), qw, s, s)


def test_reference_assertions_kept():
    """Shape asserts of the reference wrappers are kept (w4a16.py:309, quant.py:41)."""
    from kernels.quant import quantize_rtn
    from kernels.w4a16 import w4a16_matmul

    with pytest.raises(AssertionError):
        quantize_rtn(torch.randn(8, 100).half())
    with pytest.raises(AssertionError):
        w4a16_matmul(torch.randn(1, 128).half(), torch.zeros(8, 4, dtype=torch.int32),
                     torch.ones(1, 4).half(), torch.ones(1, 4).half())


@pytest.mark.skipif(torch.cuda.is_available(), reason="with a GPU, CPU tensors run there (GPU tier)")
def test_format_routines_need_a_gpu_for_cpu_tensors():
    """The weight-format routines take CPU tensors like the reference's torch code, but run them
    through the HIP kernels on a GPU: without one they raise rather than compute on the host."""
    from kernels.fp8 import dequantize_fp8, quantize_fp8
    from kernels.quant import dequantize, pack_int4, quantize_rtn, unpack_int4

    w = torch.randn(64, 128).half()
    q = torch.zeros(16, 8, dtype=torch.int32)
    for call in (lambda: quantize_rtn(w), lambda: pack_int4(q), lambda: unpack_int4(q[:2]),
                 lambda: dequantize(q[:2], torch.ones(1, 8).half(), torch.ones(1, 8).half(), 16),
                 lambda: quantize_fp8(w),
                 lambda: dequantize_fp8(torch.zeros(8, 4).to(torch.float8_e4m3fn), torch.ones(4).half())):
        with pytest.raises(RuntimeError, match="needs a ROCm GPU"):
            call()
