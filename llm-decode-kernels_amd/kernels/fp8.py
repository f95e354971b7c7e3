"""FP8 weight-only matmul (W8A16) on gfx950: y = x @ (Wq * s).T, OCP e4m3 weights.

Drop-in for the reference's `kernels/fp8.py`: weights are float8 e4m3fn with one scale per output
channel, stored [K, N] (N contiguous). gfx950 decodes OCP e4m3 natively (v_cvt_pk_f32_fp8), so
the weight bytes go straight from a 128-bit load to fp32 FMAs; the scale is applied once after
the K reduction (fp8.py:120). Quantize/dequantize run HIP kernels that reproduce the reference
bit for bit; like the reference's torch code they take CPU tensors too (run on the current ROCm
GPU, results returned on the CPU). Decode shapes run the wave64 VALU GEMV with an in-workgroup
split-K at M = 1 and the MFMA kernel (in-register byte transpose, exact e4m3 -> fp16) from 2 rows.
Prefill rows (the reference's tensor-core GEMM, fp8.py:42-91 run at fp8.py:221-222) run
hand-written kernels at every row count: the MFMA kernel in 16-row blocks (17-64 rows, and on
narrow shapes while the blocks fit in 256 workgroups: short K on 64-column tiles with K split
toward 256 workgroups, long K while they still split K at least twice), else (and from 17 rows on
wide shapes, N >= 8192) the prefill GEMM (csrc/prefill.hip: 32/64/128-row tiles, e4m3 tiles
transposed and converted to fp16 in registers, column scale after the K loop, K split over
workgroups for long K).
`config={"prefill": "gemm" | "blocks"}` forces one of them; "native" is the library's choice.
N must be a multiple of 4: rows of any such N run the VALU kernel with 4-byte loads where N % 16
!= 0, the MFMA kernel on 64-column tiles where N % 8 != 0, and the 16-row MFMA blocks instead of
the prefill GEMM where N % 16 != 0.
"""

from __future__ import annotations

import ctypes

import torch

from kernels import _lib

FP8 = torch.float8_e4m3fn
FP8_MAX = 448.0


def quantize_fp8(weight: torch.Tensor):
    """[N, K] -> (wq float8_e4m3fn [K, N], scale [N] in weight's dtype) with per-output-channel
    absmax scaling (fp8.py:25-30)."""
    N, K = weight.shape
    dev, home, (weight,) = _lib.on_gpu(weight, what="quantize_fp8")
    w = weight.contiguous()
    code = _lib.dtype_code(w.dtype)
    wq = torch.empty((K, N), dtype=FP8, device=dev)
    scale = torch.empty((N,), dtype=w.dtype, device=dev)
    with _lib.device_guard(dev):
        _lib.check(_lib.load().ldk_fp8_quantize(_lib.ptr(w), code, _lib.ptr(wq), _lib.ptr(scale),
                                                N, K, _lib.stream(dev)), "quantize_fp8")
    return wq.to(home), scale.to(home)


def dequantize_fp8(wq: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """-> [N, K] in scale's dtype (fp8.py:33-35)."""
    K, N = wq.shape
    dev, home, (wq, scale) = _lib.on_gpu(wq, scale, what="dequantize_fp8")
    code = _lib.dtype_code(scale.dtype)
    out = torch.empty((N, K), dtype=scale.dtype, device=dev)
    q = wq.contiguous()
    s = scale.contiguous()
    with _lib.device_guard(dev):
        _lib.check(_lib.load().ldk_fp8_dequant(_lib.ptr(q), _lib.ptr(s), code, _lib.ptr(out), N, K,
                                               _lib.stream(dev)), "dequantize_fp8")
    return out.to(home)


PREFILL_PATHS = ("gemm", "blocks", "native")  # "native": the library's choice


def fp8_bytes(N: int, K: int) -> int:
    """Weight bytes plus fp16 scales (fp8.py:38-39)."""
    return N * K + N * 2


def _query(M: int, N: int, K: int, block_n: int, split_k: int, flags: int):
    """(status, (block_n, split_k, flags)) of the library's plan query for ldk_w8a16_matmul."""
    bn, sk, fl = ctypes.c_int(block_n), ctypes.c_int(split_k), ctypes.c_int(flags)
    st = _lib.load().ldk_w8a16_config(M, N, K, ctypes.byref(bn), ctypes.byref(sk), ctypes.byref(fl))
    return st, (bn.value, sk.value, fl.value)


def _tuning(config: dict | None, M: int, N: int, K: int) -> tuple[int, int, int]:
    """(block_n, split_k, flags) of a call's `config`: this build's keys (`GEMV`, `MFMA`,
    `prefill`, `block_n`, `split_k`) as given; the reference's `SPLIT_K` maps onto `split_k` and
    its `BLOCK_N` onto `block_n` where the kernel the call runs takes that width (the library's
    plan query says), as in kernels.w4a16; other Triton keys are ignored."""
    cfg = config or {}
    prefill = cfg.get("prefill")
    if prefill is not None and prefill not in PREFILL_PATHS:
        raise ValueError(f"w8a16_matmul: config['prefill']={prefill!r}, expected one of {PREFILL_PATHS}")
    flags = _lib.PATH_VALU if cfg.get("GEMV") else 0
    if cfg.get("MFMA") or (M > 16 and prefill == "blocks"):
        flags |= _lib.PATH_MFMA
    elif M > 16 and prefill == "gemm":
        flags |= _lib.PATH_GEMM
    split_k = int(cfg["split_k"] if "split_k" in cfg else cfg.get("SPLIT_K", 0))
    block_n = int(cfg.get("block_n", 0))
    if "block_n" not in cfg and cfg.get("BLOCK_N"):
        want = int(cfg["BLOCK_N"])
        if _query(M, N, K, want, split_k, flags)[0] == _lib.OK:
            block_n = want
    return block_n, split_k, flags


def config_for(M: int, N: int, K: int, config: dict | None = None) -> str:
    """What ldk_w8a16_matmul runs for a shape (and `config`), as 'path,block_n=..,split_k=..'
    (the library's plan query; no GPU needed). Raises as the call would for a refused config."""
    st, (bn, sk, fl) = _query(M, N, K, *_tuning(config, M, N, K))
    _lib.check(st, "w8a16_config")
    path = "gemm" if fl & _lib.PATH_GEMM else "mfma" if fl & _lib.PATH_MFMA else "valu"
    return f"{path},block_n={bn},split_k={sk}"


def w8a16_matmul(x, wq, scale, bias=None, config=None):
    """y = x @ (wq * scale).T (+ bias). x: [..., K] fp16, wq: float8 [K, N], scale: fp16 [N]
    (fp8.py:200-223). N % 4 == 0 (the reference's column masks take any N; N = 40 in its tests).
    `config` honours `GEMV` (force the VALU kernel), `MFMA` (force the MFMA kernel), `prefill`
    (see PREFILL_PATHS), `block_n` and `split_k`, and maps the reference's `SPLIT_K` and `BLOCK_N`
    (see _tuning); other Triton tile keys are ignored."""
    K = x.shape[-1]
    N = wq.shape[1]
    assert wq.shape[0] == K
    dev = _lib.require_gpu(x, wq, scale, bias, what="w8a16_matmul")
    if x.dtype != torch.float16 or scale.dtype != torch.float16:
        raise ValueError("w8a16_matmul: x and scale must be float16")
    x2 = x.reshape(-1, K)
    if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    M = x2.shape[0]
    q = wq if wq.is_contiguous() else wq.contiguous()
    s = scale.contiguous()
    b = None if bias is None else bias.to(torch.float16).contiguous()
    block_n, split_k, flags = _tuning(config, M, N, K)
    out = torch.empty((M, N), dtype=torch.float16, device=dev)
    with _lib.device_guard(dev):
        ws, ws_bytes = _lib.workspace(dev)
        st = _lib.load().ldk_w8a16_matmul(
            _lib.ptr(x2), x2.stride(0), _lib.ptr(q), _lib.ptr(s), _lib.ptr(b), _lib.ptr(out),
            out.stride(0), M, N, K, block_n, split_k, flags, ws, ws_bytes, _lib.stream(dev))
    _lib.check(st, "w8a16_matmul")
    return out.view(*x.shape[:-1], N)
