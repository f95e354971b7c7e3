"""Writes the committed golden fixtures of the hot path (tests/golden/*.npz) from seeded inputs.

Expected outputs come from the oracle (`oracle/`, the numpy restatement of the reference's
kernels/quant.py, kernels/reference.py and kernels/fp8.py), whose every function is pinned by
known answers, invariants and brute force in tests/test_oracle_*.py. The fixtures freeze those
outputs: tests/test_golden.py checks that the oracle still reproduces them (CPU) and that the
HIP kernels match them (GPU), bit for bit where the contract is bit-exact.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import fp8 as of  # noqa: E402
from oracle import quant as oq  # noqa: E402
from oracle.reference import dequantize_ref, rmsnorm_ref, swiglu_ref, w4a16_ref  # noqa: E402


def rng(seed):
    return np.random.default_rng(seed)


def w4a16_fixture():
    g = rng(10)
    N, K, gs = 128, 256, 128
    w = (g.standard_normal((N, K), dtype=np.float32) * 0.02).astype(np.float16)
    x = g.standard_normal((4, K), dtype=np.float32).astype(np.float16)
    bias = (g.standard_normal(N, dtype=np.float32) * 0.1).astype(np.float16)
    qw, s, z = oq.quantize_rtn(w, gs)
    return dict(w=w, x=x, bias=bias, qweight=qw, scales=s, zeros=z,
                deq=dequantize_ref(qw, s, z, gs), y1=w4a16_ref(x[:1], qw, s, z, gs),
                y4_bias=w4a16_ref(x, qw, s, z, gs, bias))


def norm_act_fixture():
    g = rng(11)
    x = g.standard_normal((4, 1536), dtype=np.float32).astype(np.float16)
    r = g.standard_normal((4, 1536), dtype=np.float32).astype(np.float16)
    w = (1 + 0.1 * g.standard_normal(1536, dtype=np.float32)).astype(np.float16)
    out_res, res = rmsnorm_ref(x, w, 1e-6, residual=r)
    out = rmsnorm_ref(x, w, 1e-6)
    gu = g.standard_normal((4, 1024), dtype=np.float32).astype(np.float16)
    act = swiglu_ref(gu[:, :512], gu[:, 512:])
    return dict(x=x, r=r, w=w, out_res=out_res, res=res, out=out, gate_up=gu, act=act)


def fp8_fixture():
    g = rng(12)
    N, K = 128, 256
    w = (g.standard_normal((N, K), dtype=np.float32) * 0.02).astype(np.float16)
    x = g.standard_normal((4, K), dtype=np.float32).astype(np.float16)
    wq, s = of.quantize_fp8(w)
    return dict(w=w, x=x, wq=wq, scale=s, deq=of.dequantize_fp8(wq, s), y4=of.w8a16_ref(x, wq, s))


FIXTURES = {"w4a16": w4a16_fixture, "norm_act": norm_act_fixture, "fp8": fp8_fixture}


def main():
    for name, fn in FIXTURES.items():
        np.savez_compressed(HERE / f"{name}.npz", **fn())
        print("wrote", HERE / f"{name}.npz")


if __name__ == "__main__":
    main()
