"""Seeded synthetic inputs of the benchmark configurations (CPU torch.Generator, so the GPU run,
the parity tests and the CPU baseline see the same numbers). Recipes follow the reference's case
generators (kernels/bench/sweep.py:139-192) and tests (tests/test_w4a16.py:18-23,
tests/test_rmsnorm.py:18-22, tests/test_fp8.py:15-19): fp32 N(0, 0.02) weights cast to fp16
before quantization, N(0, 1) fp16 activations, weight drawn first, then x.
"""

from __future__ import annotations

import torch

QWEN_LINEARS = [  # (name, N, K) of Qwen2.5-1.5B, configs 2 and 3
    ("q", 1536, 1536), ("k", 256, 1536), ("v", 256, 1536), ("o", 1536, 1536),
    ("gate_up", 17920, 1536), ("down", 1536, 8960),
]


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def linear_weight(N: int, K: int, g: torch.Generator) -> torch.Tensor:
    """fp16 [N, K] ~ N(0, 0.02): drawn in fp32, then cast (sweep.py:161)."""
    return (torch.randn(N, K, generator=g) * 0.02).half()


def activations(M: int, K: int, g: torch.Generator) -> torch.Tensor:
    return torch.randn(M, K, generator=g).half()


def w4a16_case(M: int, N: int, K: int, seed: int):
    """(W fp16 [N, K], x fp16 [M, K]) on the CPU; config 0 is w4a16_case(1, 17920, 1536, 0)."""
    g = gen(seed)
    w = linear_weight(N, K, g)
    x = activations(M, K, g)
    return w, x


def rmsnorm_case(M: int, N: int, seed: int):
    """x, residual ~ N(0, 1) fp16 [M, N]; weight = 1 + 0.1 N(0, 1) in fp16 (config 1)."""
    g = gen(seed)
    x = torch.randn(M, N, generator=g).half()
    r = torch.randn(M, N, generator=g).half()
    w = (1 + 0.1 * torch.randn(N, generator=g)).half()
    return x, r, w


def swiglu_case(M: int, I: int, seed: int):
    """gate_up ~ N(0, 1) fp16 [M, 2I] (config 1)."""
    return torch.randn(M, 2 * I, generator=gen(seed)).half()
