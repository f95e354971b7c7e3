"""Greedy decode bookkeeping on the GPU: argmax of the last logits row, then out[pos] = idx,
tok = idx, pos += 1, as one HIP launch (libldk_amd.so `ldk_greedy_step`).

This is the greedy step of the reference's GraphDecoder (kernels/e2e/run.py:69-74). It replaces
`logits.argmax(-1)` inside captured decode graphs: torch's vocabulary-sized argmax reduces across
workgroups through a semaphore buffer cleared with a memset node, which is not reliable under
repeated hipGraph replay on this platform.
"""

from __future__ import annotations

import torch

from kernels import _lib


def greedy_step(logits: torch.Tensor, tok: torch.Tensor, pos: torch.Tensor,
                out: torch.Tensor | None = None) -> None:
    """logits: [..., V] (the last row is used); tok: int64 tensor of one element; pos: int64
    tensor of one element; out: optional int64 [L] token log. Updates tok, out and pos in place."""
    V = logits.shape[-1]
    row = logits.reshape(-1, V)[-1]
    if row.stride(0) != 1:
        row = row.contiguous()
    for t, name in ((tok, "tok"), (pos, "pos")):
        if t.dtype != torch.int64 or t.numel() != 1:
            raise ValueError(f"greedy_step: {name} must be one int64 element")
    if out is not None and (out.dtype != torch.int64 or not out.is_contiguous()):
        raise ValueError("greedy_step: out must be a contiguous int64 tensor")
    dev = _lib.require_gpu(row, tok, pos, out, what="greedy_step")
    with _lib.device_guard(dev):
        st = _lib.load().ldk_greedy_step(
            _lib.ptr(row), _lib.dtype_code(row.dtype), V, _lib.ptr(tok), _lib.ptr(out),
            0 if out is None else out.numel(), _lib.ptr(pos), _lib.stream(dev))
    _lib.check(st, "greedy_step")
