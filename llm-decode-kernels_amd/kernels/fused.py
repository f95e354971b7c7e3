"""Fusions on either side of the decode GEMVs (libldk_amd.so `ldk_w4a16_rmsnorm_matmul`,
`ldk_w4a16_swiglu_matmul`, `ldk_w4a16_matmul_residual_stats` + `ldk_w4a16_rmsnorm_stats_matmul`,
`ldk_w8a16_rmsnorm_matmul`, `ldk_w8a16_swiglu_matmul`).

The reference's OursBackend runs a decode layer as separate kernels: rmsnorm (+ residual), then
the W4A16 projection; swiglu, then the down projection (kernels/e2e/model.py:79-97). Here the
activation row is formed inside the W4A16 M = 1 kernel while it stages x, so each pair is one
launch. The staged activations follow the standalone kernels' rounding steps (`kernels.rmsnorm`,
`kernels.swiglu`); SwiGLU's are bit-identical to them, RMSNorm's can differ from them by one fp16
ulp, because the row's sum of squares is reduced in another order.

Rows other than one (prefill) and group sizes other than 128 run the two ops back to back.
"""

from __future__ import annotations

import torch

from kernels import _lib
from kernels.rmsnorm import rmsnorm
from kernels.swiglu import swiglu_fused
from kernels.w4a16 import w4a16_matmul

FUSED_GROUP_SIZE = 128
# Widest projection that rmsnorm_w4a16_matmul fuses. Every workgroup of the fused launch forms
# the row statistic itself (its own loads and a barrier) and the launch takes whole column tiles,
# which costs little on one round of tiles and grows with the rounds: graph-timed at K = 1536,
# N = 2048 3.46 against 3.37 us plain, N = 17920 7.52 against 5.25, and the 151936-row quantized
# lm_head 33.4 against 24.0 us, where the norm as a launch of its own (about 2.5 us) wins.
FUSED_NORM_MAX_N = 65536


def _aligned(*ts) -> bool:
    return all(t is None or (t.is_contiguous() and t.data_ptr() % 16 == 0) for t in ts)


def rmsnorm_w4a16_matmul(x, weight, eps, residual, qweight, scales, zeros, group_size=128,
                         bias=None):
    """y = w4a16_matmul(rmsnorm(x, weight, eps, residual), W) (+ bias).

    Returns (y, x + residual) when a residual is given (the updated residual stream, as
    `rmsnorm` returns it), else (y, None). x, residual: [..., K] fp16."""
    K = x.shape[-1]
    N = qweight.shape[1]
    rows = x.numel() // K
    fuse = (rows == 1 and group_size == FUSED_GROUP_SIZE and x.dtype == torch.float16
            and weight.dtype == torch.float16 and x.is_cuda and N <= FUSED_NORM_MAX_N
            and _aligned(x, weight, residual, qweight))
    if not fuse:
        if residual is None:
            h, res = rmsnorm(x, weight, eps), None
        else:
            h, res = rmsnorm(x, weight, eps, residual=residual)
        return w4a16_matmul(h, qweight, scales, zeros, group_size, bias), res
    assert qweight.shape[0] * 8 == K and weight.numel() == K
    dev = _lib.require_gpu(x, weight, residual, qweight, scales, zeros, bias,
                           what="rmsnorm_w4a16_matmul")
    if scales.dtype != torch.float16 or zeros.dtype != torch.float16:
        raise ValueError("rmsnorm_w4a16_matmul: scales and zeros must be float16")
    if residual is not None and residual.shape != x.shape:
        raise ValueError("rmsnorm_w4a16_matmul: residual must have x's shape")
    s, z = scales.contiguous(), zeros.contiguous()
    b = None if bias is None else bias.to(torch.float16).contiguous()
    out = torch.empty((*x.shape[:-1], N), dtype=torch.float16, device=dev)
    res_out = None if residual is None else torch.empty_like(x)
    with _lib.device_guard(dev):
        ws, ws_bytes = _lib.workspace(dev)
        st = _lib.load().ldk_w4a16_rmsnorm_matmul(
            _lib.ptr(x), _lib.ptr(residual), _lib.ptr(res_out), _lib.ptr(weight), float(eps),
            _lib.ptr(qweight), _lib.ptr(s), _lib.ptr(z), _lib.ptr(b), _lib.ptr(out), N, K,
            group_size, ws, ws_bytes, _lib.stream(dev))
    _lib.check(st, "rmsnorm_w4a16_matmul")
    return out, res_out


def swiglu_w4a16_matmul(gate_up, qweight, scales, zeros, group_size=128, bias=None):
    """y = w4a16_matmul(swiglu_fused(gate_up), W) (+ bias); gate_up: [..., 2K] fp16."""
    K2 = gate_up.shape[-1]
    K = K2 // 2
    N = qweight.shape[1]
    rows = gate_up.numel() // K2
    fuse = (rows == 1 and group_size == FUSED_GROUP_SIZE and gate_up.dtype == torch.float16
            and gate_up.is_cuda and _aligned(gate_up, qweight) and K % 8 == 0)
    if not fuse:
        return w4a16_matmul(swiglu_fused(gate_up), qweight, scales, zeros, group_size, bias)
    assert K2 % 2 == 0 and qweight.shape[0] * 8 == K
    dev = _lib.require_gpu(gate_up, qweight, scales, zeros, bias, what="swiglu_w4a16_matmul")
    if scales.dtype != torch.float16 or zeros.dtype != torch.float16:
        raise ValueError("swiglu_w4a16_matmul: scales and zeros must be float16")
    s, z = scales.contiguous(), zeros.contiguous()
    b = None if bias is None else bias.to(torch.float16).contiguous()
    out = torch.empty((*gate_up.shape[:-1], N), dtype=torch.float16, device=dev)
    with _lib.device_guard(dev):
        ws, ws_bytes = _lib.workspace(dev)
        st = _lib.load().ldk_w4a16_swiglu_matmul(
            _lib.ptr(gate_up), _lib.ptr(qweight), _lib.ptr(s), _lib.ptr(z), _lib.ptr(b),
            _lib.ptr(out), N, K, group_size, ws, ws_bytes, _lib.stream(dev))
    _lib.check(st, "swiglu_w4a16_matmul")
    return out


def linear_rmsnorm_w4a16_matmul(x, qweight1, scales1, zeros1, bias1, residual, weight, eps,
                                qweight2, scales2, zeros2, bias2=None, group_size=128):
    """The pair linear -> rmsnorm(+ residual) -> linear of a decoder layer (o_proj,
    post_attention_layernorm, gate_up: kernels/e2e/model.py:226-233 of the reference).

    Returns (y2, h) with h = linear1(x) + residual, the updated residual stream, and
    y2 = linear2(rmsnorm(h) * weight). One row runs two launches
    (ldk_w4a16_matmul_residual_stats, ldk_w4a16_rmsnorm_stats_matmul): the residual add and the
    row's per-tile sums of squares come out of the first projection's epilogue, so the second
    one forms the norm in its x staging without reducing the row itself. Other rows run
    w4a16_matmul then rmsnorm_w4a16_matmul."""
    K1 = x.shape[-1]
    N1 = qweight1.shape[1]
    rows = x.numel() // K1
    fuse = (rows == 1 and group_size == FUSED_GROUP_SIZE and x.dtype == torch.float16 and x.is_cuda
            and residual is not None and residual.dtype == torch.float16
            and residual.numel() == N1 and weight.dtype == torch.float16
            and _aligned(x, residual, weight, qweight1, qweight2))
    nstats = int(_lib.load().ldk_w4a16_row_stats_count(N1, K1, group_size)) if fuse else 0
    if not fuse or not 0 < nstats <= 256:
        y1 = w4a16_matmul(x, qweight1, scales1, zeros1, group_size, bias1)
        return rmsnorm_w4a16_matmul(y1, weight, eps, residual, qweight2, scales2, zeros2,
                                    group_size, bias2)
    K2, N2 = N1, qweight2.shape[1]
    assert qweight1.shape[0] * 8 == K1 and qweight2.shape[0] * 8 == K2 and weight.numel() == K2
    dev = _lib.require_gpu(x, residual, weight, qweight1, scales1, zeros1, bias1, qweight2,
                           scales2, zeros2, bias2, what="linear_rmsnorm_w4a16_matmul")
    for t in (scales1, zeros1, scales2, zeros2):
        if t.dtype != torch.float16:
            raise ValueError("linear_rmsnorm_w4a16_matmul: scales and zeros must be float16")
    b1 = None if bias1 is None else bias1.to(torch.float16).contiguous()
    b2 = None if bias2 is None else bias2.to(torch.float16).contiguous()
    s1, z1, s2, z2 = (t.contiguous() for t in (scales1, zeros1, scales2, zeros2))
    h = torch.empty((*x.shape[:-1], N1), dtype=torch.float16, device=dev)
    stats = torch.empty(nstats, dtype=torch.float32, device=dev)
    y2 = torch.empty((*x.shape[:-1], N2), dtype=torch.float16, device=dev)
    lib = _lib.load()
    with _lib.device_guard(dev):
        ws, ws_bytes = _lib.workspace(dev)
        st = lib.ldk_w4a16_matmul_residual_stats(
            _lib.ptr(x), _lib.ptr(residual), _lib.ptr(h), _lib.ptr(stats), _lib.ptr(qweight1),
            _lib.ptr(s1), _lib.ptr(z1), _lib.ptr(b1), N1, K1,
            group_size, ws, ws_bytes, _lib.stream(dev))
        _lib.check(st, "linear_rmsnorm_w4a16_matmul")
        st = lib.ldk_w4a16_rmsnorm_stats_matmul(
            _lib.ptr(h), _lib.ptr(stats), nstats, _lib.ptr(weight), float(eps), _lib.ptr(qweight2),
            _lib.ptr(s2), _lib.ptr(z2), _lib.ptr(b2),
            _lib.ptr(y2), N2, K2, group_size, ws, ws_bytes, _lib.stream(dev))
        _lib.check(st, "linear_rmsnorm_w4a16_matmul")
    return y2, h


def attn_linear_rmsnorm_w4a16_matmul(ranges, qweight1, scales1, zeros1, bias1, residual, weight,
                                     eps, qweight2, scales2, zeros2, bias2=None, group_size=128):
    """linear_rmsnorm_w4a16_matmul with x the decode attention output that
    kernels.attention.decode_attention_ranges left as per-range partials (`ranges`): the first
    projection merges the ranges in its x staging (ldk_w4a16_attn_matmul_residual_stats), so the
    attention's merge launch and the o projection are one launch. Returns (y2, h) as
    linear_rmsnorm_w4a16_matmul does. One row, group size 128, K1 = 128 * heads, at most four
    ranges."""
    K1 = qweight1.shape[0] * 8
    N1 = qweight1.shape[1]
    if group_size != FUSED_GROUP_SIZE:
        raise ValueError(f"attn_linear_rmsnorm_w4a16_matmul: group_size {group_size} (fused: 128)")
    if K1 != 128 * ranges.n_heads:
        raise ValueError("attn_linear_rmsnorm_w4a16_matmul: K must be 128 * the attention's heads")
    if residual.dtype != torch.float16 or residual.numel() != N1 or weight.dtype != torch.float16:
        raise ValueError("attn_linear_rmsnorm_w4a16_matmul: fp16 residual of N1 values and weight")
    # the C entry reads qweight1/qweight2 as packed [K/8, N] and the norm weight as [K2], each
    # with 16-byte loads: a strided view would be read as the wrong elements
    if not _aligned(qweight1, qweight2, weight):
        raise ValueError("attn_linear_rmsnorm_w4a16_matmul: qweight1, qweight2 and weight must be "
                         "contiguous and 16-byte aligned")
    K2, N2 = N1, qweight2.shape[1]
    assert qweight2.shape[0] * 8 == K2 and weight.numel() == K2
    dev = _lib.require_gpu(ranges.pos, residual, weight, qweight1, scales1, zeros1, bias1, qweight2,
                           scales2, zeros2, bias2, what="attn_linear_rmsnorm_w4a16_matmul")
    for t in (scales1, zeros1, scales2, zeros2):
        if t.dtype != torch.float16:
            raise ValueError("attn_linear_rmsnorm_w4a16_matmul: scales and zeros must be float16")
    nstats = int(_lib.load().ldk_w4a16_row_stats_count(N1, K1, group_size))
    if not 0 < nstats <= 256:
        raise ValueError(f"attn_linear_rmsnorm_w4a16_matmul: {nstats} row partials (1..256)")
    b1 = None if bias1 is None else bias1.to(torch.float16).contiguous()
    b2 = None if bias2 is None else bias2.to(torch.float16).contiguous()
    s1, z1, s2, z2 = (t.contiguous() for t in (scales1, zeros1, scales2, zeros2))
    r = residual if residual.is_contiguous() else residual.contiguous()
    h = torch.empty(residual.shape, dtype=torch.float16, device=dev)
    stats = torch.empty(nstats, dtype=torch.float32, device=dev)
    y2 = torch.empty((*residual.shape[:-1], N2), dtype=torch.float16, device=dev)
    lib = _lib.load()
    with _lib.device_guard(dev):
        ws, ws_bytes = _lib.workspace(dev)
        st = lib.ldk_w4a16_attn_matmul_residual_stats(
            _lib.ptr(ranges.pos), ranges.max_len, ranges.rlen, ranges.n_heads, _lib.ptr(r),
            _lib.ptr(h), _lib.ptr(stats), _lib.ptr(qweight1), _lib.ptr(s1), _lib.ptr(z1),
            _lib.ptr(b1), N1, K1, group_size, ws, ws_bytes, _lib.stream(dev))
        _lib.check(st, "attn_linear_rmsnorm_w4a16_matmul")
        st = lib.ldk_w4a16_rmsnorm_stats_matmul(
            _lib.ptr(h), _lib.ptr(stats), nstats, _lib.ptr(weight), float(eps), _lib.ptr(qweight2),
            _lib.ptr(s2), _lib.ptr(z2), _lib.ptr(b2),
            _lib.ptr(y2), N2, K2, group_size, ws, ws_bytes, _lib.stream(dev))
        _lib.check(st, "attn_linear_rmsnorm_w4a16_matmul")
    return y2, h


def w4a16_matmul_swiglu(x, qweight, scales, zeros, group_size=128, bias=None):
    """swiglu_fused(w4a16_matmul(x, W) (+ bias)) for prefill rows, x [..., K] fp16 -> [..., N/2]:
    one launch where the library's plan for the shape is the prefill GEMM on paired column groups
    (ldk_w4a16_matmul_swiglu: the g and u halves of the product meet in the GEMM's epilogue), else
    the two ops; bit for bit the two ops either way."""
    K = x.shape[-1]
    N = qweight.shape[1]
    rows = x.numel() // K
    fuse = (rows > 16 and x.dtype == torch.float16 and x.is_cuda and N % 2 == 0
            and _aligned(x, qweight)
            and bool(_lib.load().ldk_w4a16_matmul_swiglu_applies(rows, N, K, group_size)))
    if not fuse:
        return swiglu_fused(w4a16_matmul(x, qweight, scales, zeros, group_size, bias))
    assert qweight.shape[0] * 8 == K
    dev = _lib.require_gpu(x, qweight, scales, zeros, bias, what="w4a16_matmul_swiglu")
    if scales.dtype != torch.float16 or zeros.dtype != torch.float16:
        raise ValueError("w4a16_matmul_swiglu: scales and zeros must be float16")
    s, z = scales.contiguous(), zeros.contiguous()
    b = None if bias is None else bias.to(torch.float16).contiguous()
    out = torch.empty((*x.shape[:-1], N // 2), dtype=torch.float16, device=dev)
    with _lib.device_guard(dev):
        ws, ws_bytes = _lib.workspace(dev)
        st = _lib.load().ldk_w4a16_matmul_swiglu(
            _lib.ptr(x), K, _lib.ptr(qweight), _lib.ptr(s), _lib.ptr(z), _lib.ptr(b), _lib.ptr(out), N // 2,
            rows, N, K, group_size, ws, ws_bytes, _lib.stream(dev))
    _lib.check(st, "w4a16_matmul_swiglu")
    return out


def w8a16_matmul_swiglu(x, wq, scale, bias=None):
    """swiglu_fused(w8a16_matmul(x, wq, scale) (+ bias)) for prefill rows, x [..., K] fp16, wq
    [K, N] float8_e4m3fn -> [..., N/2]: one launch where the library's plan for the shape is the
    prefill GEMM on paired column groups (ldk_w8a16_matmul_swiglu), else the two ops; bit for bit
    the two ops either way."""
    from kernels.fp8 import FP8, w8a16_matmul

    K = x.shape[-1]
    N = wq.shape[1]
    rows = x.numel() // K
    fuse = (rows > 16 and x.dtype == torch.float16 and x.is_cuda and N % 2 == 0 and wq.dtype == FP8
            and scale.dtype == torch.float16 and _aligned(x, wq)
            and bool(_lib.load().ldk_w8a16_matmul_swiglu_applies(rows, N, K)))
    if not fuse:
        return swiglu_fused(w8a16_matmul(x, wq, scale, bias=bias))
    assert wq.shape[0] == K
    dev = _lib.require_gpu(x, wq, scale, bias, what="w8a16_matmul_swiglu")
    s = scale.contiguous()
    b = None if bias is None else bias.to(torch.float16).contiguous()
    out = torch.empty((*x.shape[:-1], N // 2), dtype=torch.float16, device=dev)
    with _lib.device_guard(dev):
        ws, ws_bytes = _lib.workspace(dev)
        st = _lib.load().ldk_w8a16_matmul_swiglu(
            _lib.ptr(x), K, _lib.ptr(wq), _lib.ptr(s), _lib.ptr(b), _lib.ptr(out), N // 2, rows, N, K,
            ws, ws_bytes, _lib.stream(dev))
    _lib.check(st, "w8a16_matmul_swiglu")
    return out


def swiglu_w8a16_matmul(gate_up, wq, scale, bias=None):
    """y = w8a16_matmul(swiglu_fused(gate_up), wq, scale) (+ bias); gate_up: [..., 2K] fp16,
    wq: [K, N] float8_e4m3fn, scale: [N] fp16. One row runs one launch (ldk_w8a16_swiglu_matmul),
    more rows the two ops back to back."""
    from kernels.fp8 import FP8, w8a16_matmul

    K2 = gate_up.shape[-1]
    K = K2 // 2
    N = wq.shape[1]
    rows = gate_up.numel() // K2
    fuse = (rows == 1 and gate_up.dtype == torch.float16 and gate_up.is_cuda and K2 % 2 == 0
            and K % 8 == 0 and N % 4 == 0 and wq.dtype == FP8 and scale.dtype == torch.float16
            and _aligned(gate_up, wq))
    if not fuse:
        return w8a16_matmul(swiglu_fused(gate_up), wq, scale, bias=bias)
    assert wq.shape[0] == K and scale.numel() == N
    dev = _lib.require_gpu(gate_up, wq, scale, bias, what="swiglu_w8a16_matmul")
    b = None if bias is None else bias.to(torch.float16).contiguous()
    sc = scale.contiguous()
    out = torch.empty((*gate_up.shape[:-1], N), dtype=torch.float16, device=dev)
    with _lib.device_guard(dev):
        ws, ws_bytes = _lib.workspace(dev)
        st = _lib.load().ldk_w8a16_swiglu_matmul(
            _lib.ptr(gate_up), _lib.ptr(wq), _lib.ptr(sc), _lib.ptr(b), _lib.ptr(out), N, K, ws,
            ws_bytes, _lib.stream(dev))
    _lib.check(st, "swiglu_w8a16_matmul")
    return out


def rmsnorm_w8a16_matmul(x, weight, eps, residual, wq, scale, bias=None):
    """y = w8a16_matmul(rmsnorm(x, weight, eps, residual), wq, scale) (+ bias).

    Returns (y, x + residual) when a residual is given, else (y, None). One row runs one launch
    (ldk_w8a16_rmsnorm_matmul), more rows the two ops back to back."""
    from kernels.fp8 import FP8, w8a16_matmul

    K = x.shape[-1]
    N = wq.shape[1]
    rows = x.numel() // K
    fuse = (rows == 1 and x.dtype == torch.float16 and weight.dtype == torch.float16 and x.is_cuda
            and K % 8 == 0 and N % 4 == 0 and wq.dtype == FP8 and scale.dtype == torch.float16
            and _aligned(x, weight, residual, wq))
    if not fuse:
        if residual is None:
            h, res = rmsnorm(x, weight, eps), None
        else:
            h, res = rmsnorm(x, weight, eps, residual=residual)
        return w8a16_matmul(h, wq, scale, bias=bias), res
    assert wq.shape[0] == K and weight.numel() == K and scale.numel() == N
    dev = _lib.require_gpu(x, weight, residual, wq, scale, bias, what="rmsnorm_w8a16_matmul")
    if residual is not None and residual.shape != x.shape:
        raise ValueError("rmsnorm_w8a16_matmul: residual must have x's shape")
    b = None if bias is None else bias.to(torch.float16).contiguous()
    sc = scale.contiguous()
    out = torch.empty((*x.shape[:-1], N), dtype=torch.float16, device=dev)
    res_out = None if residual is None else torch.empty_like(x)
    with _lib.device_guard(dev):
        ws, ws_bytes = _lib.workspace(dev)
        st = _lib.load().ldk_w8a16_rmsnorm_matmul(
            _lib.ptr(x), _lib.ptr(residual), _lib.ptr(res_out), _lib.ptr(weight), float(eps),
            _lib.ptr(wq), _lib.ptr(sc), _lib.ptr(b), _lib.ptr(out), N, K, ws, ws_bytes,
            _lib.stream(dev))
    _lib.check(st, "rmsnorm_w8a16_matmul")
    return out, res_out


def attn_w8a16_matmul(ranges, wq, scale, bias=None):
    """y = w8a16_matmul(attention output, wq, scale) (+ bias) with the attention output the
    per-range partials kernels.attention.decode_attention_ranges left (`ranges`): the projection
    merges the ranges in its x staging (ldk_w8a16_attn_matmul), so the attention's merge launch
    and the FP8 o projection are one launch. One row, K = 128 * heads, at most four ranges.
    Returns [1, N] fp16."""
    from kernels.fp8 import FP8

    K, N = wq.shape
    if wq.dtype != FP8 or scale.dtype != torch.float16 or scale.numel() != N:
        raise ValueError("attn_w8a16_matmul: wq [K, N] float8_e4m3fn and fp16 scale [N]")
    if K != 128 * ranges.n_heads:
        raise ValueError("attn_w8a16_matmul: K must be 128 * the attention's heads")
    # the C entry reads wq as [K, N] rows with 16-byte loads: a strided view would be read as
    # the wrong elements
    if not _aligned(wq):
        raise ValueError("attn_w8a16_matmul: wq must be contiguous and 16-byte aligned")
    dev = _lib.require_gpu(ranges.pos, wq, scale, bias, what="attn_w8a16_matmul")
    b = None if bias is None else bias.to(torch.float16).contiguous()
    sc = scale.contiguous()
    out = torch.empty((1, N), dtype=torch.float16, device=dev)
    with _lib.device_guard(dev):
        ws, ws_bytes = _lib.workspace(dev)
        st = _lib.load().ldk_w8a16_attn_matmul(
            _lib.ptr(ranges.pos), ranges.max_len, ranges.rlen, ranges.n_heads, _lib.ptr(wq),
            _lib.ptr(sc), _lib.ptr(b), _lib.ptr(out), N, K, ws, ws_bytes, _lib.stream(dev))
    _lib.check(st, "attn_w8a16_matmul")
    return out


__all__ = ["rmsnorm_w4a16_matmul", "swiglu_w4a16_matmul", "linear_rmsnorm_w4a16_matmul",
           "attn_linear_rmsnorm_w4a16_matmul", "w4a16_matmul_swiglu", "w8a16_matmul_swiglu", "rmsnorm_w8a16_matmul",
           "swiglu_w8a16_matmul", "attn_w8a16_matmul"]
