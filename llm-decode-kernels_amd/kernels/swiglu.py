"""Fused SwiGLU activation on gfx950: out = silu(gate) * up, in one pass.

Drop-in for the reference's `kernels/swiglu.py`: accepts two tensors or one fused [.., 2*I]
tensor (gate first, then up) whose halves are read in place. silu is computed in fp32 and
rounded to fp16 like F.silu, then multiplied by `up` in fp16 (kernels/reference.py:22-24).
"""

from __future__ import annotations

import torch

from kernels import _lib


def _launch(gate2: torch.Tensor, up2: torch.Tensor) -> torch.Tensor:
    M, I = gate2.shape
    assert gate2.stride(-1) == 1 and up2.stride(-1) == 1
    dev = _lib.require_gpu(gate2, up2, what="swiglu")
    if gate2.dtype != torch.float16 or up2.dtype != torch.float16:
        raise ValueError("swiglu: gate and up must be float16")
    out = torch.empty((M, I), dtype=gate2.dtype, device=dev)
    with _lib.device_guard(dev):
        st = _lib.load().ldk_swiglu(_lib.ptr(gate2), gate2.stride(0), _lib.ptr(up2), up2.stride(0),
                                    _lib.ptr(out), out.stride(0), M, I, _lib.stream(dev))
    _lib.check(st, "swiglu")
    return out


def swiglu(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up for two same-shape tensors (swiglu.py:49-53)."""
    I = gate.shape[-1]
    out = _launch(gate.reshape(-1, I), up.reshape(-1, I))
    return out.view(gate.shape)


def swiglu_fused(gate_up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up where gate_up = cat([gate, up], dim=-1); reads the halves in place
    (swiglu.py:56-61)."""
    I = gate_up.shape[-1] // 2
    gu = gate_up.reshape(-1, 2 * I)
    out = _launch(gu[:, :I], gu[:, I:])
    return out.view(*gate_up.shape[:-1], I)


def swiglu_bytes(M: int, I: int, elem: int = 2) -> int:
    """Read gate and up, write out (swiglu.py:64-65)."""
    return 3 * M * I * elem
