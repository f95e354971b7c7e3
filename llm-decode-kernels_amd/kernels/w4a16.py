"""W4A16 matmul on gfx950: y = x @ dequant(W).T (+ bias), int4 weights, fp16 activations.

Drop-in for the reference's `kernels/w4a16.py` (same `w4a16_matmul` signature, same int4 format
from `kernels.quant`). Decode shapes (M <= 16) run one hand-written HIP kernel from
libldk_amd.so whose tile and K-split come from the library's per-shape table:

- each workgroup owns a strip of output columns and a range of K; lanes split K and the partial
  sums are reduced inside the workgroup (DPP/permlane within a wave, LDS across waves); narrow
  shapes with many bytes (the down projection) also split K across workgroups that meet in a
  per-device workspace, all within the one launch, so there is no zero-fill or cast launch (the
  reference's split paths add two elementwise launches, w4a16.py:218-219,272-275);
- M = 1 and M = 2 use the FACTORED inner loop s * (sum x*q - z * sum x) (w4a16.py:116-119) on
  the VALU, each packed word decoded once for both rows; from 3 rows the MFMA kernel computes the
  same factored form on the matrix cores. `config={"FACTORED": False}` (EXACT, M <= 8) instead
  dequantizes each weight exactly as dequantize_ref and accumulates with v_dot2_f32_f16.

Prefill shapes (the reference's Triton tensor-core GEMM path, w4a16.py:264-268) run hand-written
kernels at every row count: the library picks, per shape, the prefill GEMM (csrc/prefill.hip:
32/64/128-row tiles on the matrix cores, every weight dequantized exactly as dequantize_ref does
it, fp32 accumulation, K split over workgroups for long K) or the MFMA kernel in 16- or 32-row blocks
(the choice for 17-31 rows and for narrow shapes up to 256 rows, and up to 511 rows while the
blocks fit in 256 workgroups, where the blocks' K split over waves wins; 16-row blocks wherever
they fit in 256 workgroups, with K split over workgroups on long K; wide shapes, N >= 8192, take
the GEMM from 32 rows). `config={"prefill": "gemm" | "blocks"}` forces one of them; "native" is the library's choice.

`config` (dict) forces a variant, as in the reference (w4a16.py:301-306). Honoured keys:
`GEMV` (force the VALU decode kernels, M <= 8), `MFMA` (force the MFMA kernel), `FACTORED`
(True: the factored loop, on the VALU kernel for M <= 2; False: exact dequantize-then-dot on the
VALU kernels, M <= 8),
`block_n` (columns per workgroup: 16, 32 or 64; 64 or 128 on the MFMA kernel), `split_k`
(workgroups splitting K per column tile) and `chunks_per_wave` (1, 2 or 4: load chunks a wave
keeps in flight per round). Of the reference's Triton keys, `SPLIT_K` maps onto `split_k` and
`BLOCK_N` onto `block_n` where the kernel the call runs takes that width; BLOCK_M, BLOCK_K and
GROUP_M describe Triton programs and are ignored. `config_for(M, N, K, group_size, config)`
reports what a config runs.
"""

from __future__ import annotations

import ctypes

import torch

from kernels import _lib
from kernels.quant import PACK

_decode_choice: dict[tuple, str] = {}  # (m_key, N, K, bias) -> chosen configuration, for export

PREFILL_PATHS = ("gemm", "blocks", "native")  # "native": the library's choice


def _next_pow2(n: int) -> int:
    return 1 << max(0, (n - 1).bit_length())


def _query(M: int, N: int, K: int, group_size: int, block_n: int, split_k: int, flags: int):
    """(status, (block_n, split_k, flags)) of the library's plan query: what a call with these
    tuning arguments runs, or the status it would fail with."""
    bn, sk, fl = ctypes.c_int(block_n), ctypes.c_int(split_k), ctypes.c_int(flags)
    st = _lib.load().ldk_w4a16_config(M, N, K, group_size, ctypes.byref(bn), ctypes.byref(sk),
                                      ctypes.byref(fl))
    return st, (bn.value, sk.value, fl.value)


def _tuning(config: dict | None, M: int, N: int, K: int, group_size: int) -> tuple[int, int, int]:
    """(block_n, split_k, flags) of a call's `config`. This build's keys (`block_n`, `split_k`,
    `GEMV`, `MFMA`, `FACTORED`, `chunks_per_wave`, `prefill`) are passed as given. The reference's
    Triton keys map where they mean the same thing here (w4a16.py:301-330): `SPLIT_K` is the
    number of workgroups splitting K per column tile (1: no split; the groups are dealt evenly
    over exactly that many), and `BLOCK_N`, the output columns per program, becomes `block_n`
    when the kernel the call runs takes that width (checked with the library's plan query),
    else it is ignored, as are BLOCK_M, BLOCK_K and GROUP_M (Triton tile shapes)."""
    if not config:
        return 0, 0, 0
    flags = 0
    if config.get("GEMV"):
        flags |= _lib.PATH_VALU
    if config.get("MFMA"):
        flags |= _lib.PATH_MFMA
    if "FACTORED" in config:
        if config["FACTORED"] and (M <= 2 or not config.get("GEMV")):
            flags |= _lib.FACTORED
        elif not config["FACTORED"]:
            flags |= _lib.EXACT
    if config.get("chunks_per_wave"):
        flags |= _lib.CPW_FLAGS[int(config["chunks_per_wave"])]
    prefill = config.get("prefill")
    if prefill is not None and prefill not in PREFILL_PATHS:
        raise ValueError(f"w4a16_matmul: config['prefill']={prefill!r}, expected one of {PREFILL_PATHS}")
    if M > 16 and prefill == "gemm":
        flags |= _lib.PATH_GEMM
    elif M > 16 and prefill == "blocks":
        flags |= _lib.PATH_MFMA
    split_k = int(config["split_k"] if "split_k" in config else config.get("SPLIT_K", 0))
    block_n = int(config.get("block_n", 0))
    if "block_n" not in config and config.get("BLOCK_N"):
        want = int(config["BLOCK_N"])
        if _query(M, N, K, group_size, want, split_k, flags)[0] == _lib.OK:
            block_n = want
    return block_n, split_k, flags


def _decode(x2, qweight, scales, zeros, bias, group_size, block_n, split_k, flags, out):
    M, K = x2.shape
    N = qweight.shape[1]
    dev = x2.device
    with _lib.device_guard(dev):
        ws, ws_bytes = _lib.workspace(dev)
        st = _lib.load().ldk_w4a16_matmul(
            _lib.ptr(x2), x2.stride(0), _lib.ptr(qweight), _lib.ptr(scales), _lib.ptr(zeros),
            _lib.ptr(bias), _lib.ptr(out), out.stride(0), M, N, K, group_size, block_n, split_k,
            flags, ws, ws_bytes, _lib.stream(dev))
    _lib.check(st, "w4a16_matmul")
    return out


def w4a16_matmul(x, qweight, scales, zeros, group_size=128, bias=None, config=None):
    """y = x @ dequant(W).T (+ bias). x: [..., K] fp16. Returns [..., N] fp16 (w4a16.py:301-330)."""
    K = x.shape[-1]
    N = qweight.shape[1]
    assert qweight.shape[0] * 8 == K and K % group_size == 0
    dev = _lib.require_gpu(x, qweight, scales, zeros, bias, what="w4a16_matmul")
    if x.dtype != torch.float16 or scales.dtype != torch.float16 or zeros.dtype != torch.float16:
        raise ValueError("w4a16_matmul: x, scales and zeros must be float16")
    x2 = x.reshape(-1, K)
    if x2.stride(1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    M = x2.shape[0]
    qw = qweight if qweight.is_contiguous() else qweight.contiguous()
    s = scales if scales.is_contiguous() else scales.contiguous()
    z = zeros if zeros.is_contiguous() else zeros.contiguous()
    b = None if bias is None else bias.to(torch.float16).contiguous()
    block_n, split_k, flags = _tuning(config, M, N, K, group_size)
    out = torch.empty((M, N), dtype=torch.float16, device=dev)
    _decode(x2, qw, s, z, b, group_size, block_n, split_k, flags, out)
    # the library's choice is recorded for the decode shapes it chose (w4a16.py:322-326): a call
    # whose config forced a variant records nothing, as the reference's forced path picks nothing
    key = (min(_next_pow2(M), 16), N, K, bias is not None)
    if M <= 16 and not config and key not in _decode_choice:
        _decode_choice[key] = config_for(M, N, K, group_size)
    return out.view(*x.shape[:-1], N)


def config_for(M: int, N: int, K: int, group_size: int = 128, config: dict | None = None) -> str:
    """What the library runs for a shape, as 'path,block_n=..,split_k=..,mode': its table choice,
    or with `config` what a call with that config runs (the library's plan query; no GPU
    needed). Raises as the call would for a config it refuses."""
    st, (bn, sk, fl) = _query(M, N, K, group_size, *_tuning(config, M, N, K, group_size))
    _lib.check(st, "w4a16_config")
    if fl & _lib.PATH_GEMM:
        return f"gemm,block_n={bn},split_k={sk}"
    mode = "factored" if fl & _lib.FACTORED else "exact"
    path = "mfma" if fl & _lib.PATH_MFMA else "valu"
    cpw = {v: k for k, v in _lib.CPW_FLAGS.items()}.get(fl & _lib.CPW_MASK)
    extra = f",chunks_per_wave={cpw}" if cpw else ""
    return f"{path},block_n={bn},split_k={sk},{mode}{extra}"


def kernel_name(M: int, N: int, K: int, group_size: int = 128) -> str:
    """The kernel instantiation the library runs for a shape, as the profiler names it."""
    buf = ctypes.create_string_buffer(256)
    _lib.check(_lib.load().ldk_w4a16_kernel_name(M, N, K, group_size, buf, len(buf)),
               "w4a16_kernel_name")
    return buf.value.decode()


def export_choices() -> dict:
    """Configurations used so far (w4a16.py:333-335)."""
    return {",".join(map(str, k)): v for k, v in _decode_choice.items()}


def import_choices(choices: dict) -> None:
    """Accepts an export_choices() dict (w4a16.py:338-342). The library's choice is a pure
    function of the shape, so importing only records the entries."""
    for k, v in choices.items():
        m, n, kk, b = k.split(",")
        _decode_choice[(int(m), int(n), int(kk), b == "True")] = v


def best_configs() -> dict:
    """Configurations used so far, for the results JSON (w4a16.py:345-355)."""
    return {"decode_path": {str(k): v for k, v in _decode_choice.items()}}


__all__ = ["w4a16_matmul", "export_choices", "import_choices", "best_configs", "config_for",
           "kernel_name", "PACK"]
