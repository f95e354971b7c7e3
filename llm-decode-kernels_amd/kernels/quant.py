"""4-bit weight format shared by every kernel in this package, produced on the GPU.

Same layout and names as the reference's `kernels/quant.py` (lines 3-10): for a linear layer with
weight W of shape [N, K] (out_features, in_features)

- `qweight`: int32 [K // 8, N]. Each int32 holds 8 consecutive K values of one output column,
  value i in bits 4i..4i+3 (0..15). N is the contiguous dimension.
- `scales`, `zeros`: [K // group_size, N] in the weight's dtype. Dequantized weight:
  (q - zero) * scale.

Quantization is round-to-nearest (RTN), asymmetric, group size 128 along K. Every function here
runs a HIP kernel (libldk_amd.so) and reproduces the reference bit for bit. Like the reference's
device-agnostic torch code, each accepts CPU tensors (run on the current ROCm GPU, results
returned on the CPU) or GPU tensors.
"""

from __future__ import annotations

import torch

from kernels import _lib

PACK = 8  # int4 values per int32 (quant.py:17)


def pack_int4(q: torch.Tensor) -> torch.Tensor:
    """[K, N] integers in 0..15 -> [K // 8, N] int32 (quant.py:20-28)."""
    K, N = q.shape
    assert K % PACK == 0, "K must be a multiple of 8"
    dev, home, (q,) = _lib.on_gpu(q, what="pack_int4")
    q32 = q.to(torch.int32).contiguous()
    out = torch.empty((K // PACK, N), dtype=torch.int32, device=dev)
    with _lib.device_guard(dev):
        _lib.check(_lib.load().ldk_int4_pack(_lib.ptr(q32), _lib.ptr(out), K, N, _lib.stream(dev)),
                   "pack_int4")
    return out.to(home)


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    """[K // 8, N] int32 -> [K, N] int32 in 0..15 (quant.py:31-35)."""
    assert packed.dtype == torch.int32 and packed.dim() == 2
    dev, home, (packed,) = _lib.on_gpu(packed, what="unpack_int4")
    p = packed.contiguous()
    R, N = p.shape
    out = torch.empty((R * PACK, N), dtype=torch.int32, device=dev)
    with _lib.device_guard(dev):
        _lib.check(_lib.load().ldk_int4_unpack(_lib.ptr(p), _lib.ptr(out), R * PACK, N,
                                               _lib.stream(dev)), "unpack_int4")
    return out.to(home)


def quantize_rtn(weight: torch.Tensor, group_size: int = 128):
    """Round-to-nearest asymmetric int4 quantization of an [N, K] weight (quant.py:38-49).

    Returns (qweight int32 [K/8, N], scales [K/G, N], zeros [K/G, N]); scales and zeros have the
    weight's dtype (fp16 for an fp16 weight), exactly as the reference returns them."""
    N, K = weight.shape
    assert K % group_size == 0, f"K={K} must be a multiple of group_size={group_size}"
    dev, home, (weight,) = _lib.on_gpu(weight, what="quantize_rtn")
    w = weight.contiguous()
    code = _lib.dtype_code(w.dtype)
    qweight = torch.empty((K // PACK, N), dtype=torch.int32, device=dev)
    scales = torch.empty((K // group_size, N), dtype=w.dtype, device=dev)
    zeros = torch.empty_like(scales)
    with _lib.device_guard(dev):
        _lib.check(_lib.load().ldk_quantize_rtn(
            _lib.ptr(w), code, _lib.ptr(qweight), _lib.ptr(scales), _lib.ptr(zeros), N, K,
            group_size, _lib.stream(dev)), "quantize_rtn")
    return qweight.to(home), scales.to(home), zeros.to(home)


def dequantize(qweight: torch.Tensor, scales: torch.Tensor, zeros: torch.Tensor,
               group_size: int = 128) -> torch.Tensor:
    """int4 -> fp16 [N, K] (nn.Linear layout), one fp16 rounding of (q - z) * s: bit-identical to
    the reference's dequantize_ref (kernels/reference.py:27-36)."""
    R, N = qweight.shape
    K = R * PACK
    assert K % group_size == 0 and scales.shape == (K // group_size, N) == zeros.shape
    assert scales.dtype == torch.float16 and zeros.dtype == torch.float16, "fp16 scales/zeros"
    dev, home, (qweight, scales, zeros) = _lib.on_gpu(qweight, scales, zeros, what="dequantize")
    out = torch.empty((N, K), dtype=torch.float16, device=dev)
    qw, s, z = qweight.contiguous(), scales.contiguous(), zeros.contiguous()
    with _lib.device_guard(dev):
        _lib.check(_lib.load().ldk_w4a16_dequant(
            _lib.ptr(qw), _lib.ptr(s), _lib.ptr(z), _lib.ptr(out), N, K, group_size,
            _lib.stream(dev)), "dequantize")
    return out.to(home)


def weight_bytes(N: int, K: int, group_size: int = 128) -> int:
    """Bytes a W4A16 kernel must read for the weight: packed int4 + fp16 scales and zeros
    (quant.py:52-54)."""
    return N * K // 2 + 2 * (K // group_size) * N * 2
