"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU tier: the oracle still reproduces every frozen output from the frozen inputs, bit for bit.
GPU tier: the HIP kernels match the frozen outputs, with the north-star bars: int4 format,
dequantization, FP8 quantization and the residual bit-exact; matmul outputs within max-abs 2e-2
and relative-L2 1e-3; RMSNorm and SwiGLU within one fp16 ulp of the rounded intermediate."""

from pathlib import Path

import numpy as np
import pytest
import torch

from _util import assert_north_star, bits16, dev, to_np
from oracle import fp8 as of
from oracle import quant as oq
from oracle.reference import dequantize_ref, rmsnorm_ref, swiglu_ref, w4a16_ref

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


def test_fixture_sizes():
    """Small data, committed: the three fixtures stay under 512 KB together."""
    assert sum(p.stat().st_size for p in GOLDEN.glob("*.npz")) < 512 * 1024


def test_oracle_reproduces_w4a16_fixture():
    g = load("w4a16")
    qw, s, z = oq.quantize_rtn(g["w"], 128)
    assert np.array_equal(qw, g["qweight"])
    assert np.array_equal(bits16(s), bits16(g["scales"])) and np.array_equal(bits16(z), bits16(g["zeros"]))
    assert np.array_equal(bits16(dequantize_ref(qw, s, z)), bits16(g["deq"]))
    assert np.array_equal(w4a16_ref(g["x"][:1], qw, s, z), g["y1"])
    assert np.array_equal(w4a16_ref(g["x"], qw, s, z, 128, g["bias"]), g["y4_bias"])


def test_oracle_reproduces_norm_act_fixture():
    g = load("norm_act")
    out, res = rmsnorm_ref(g["x"], g["w"], 1e-6, residual=g["r"])
    assert np.array_equal(bits16(out), bits16(g["out_res"])) and np.array_equal(bits16(res), bits16(g["res"]))
    assert np.array_equal(bits16(rmsnorm_ref(g["x"], g["w"], 1e-6)), bits16(g["out"]))
    gu = g["gate_up"]
    assert np.array_equal(bits16(swiglu_ref(gu[:, :512], gu[:, 512:])), bits16(g["act"]))


def test_oracle_reproduces_fp8_fixture():
    g = load("fp8")
    wq, s = of.quantize_fp8(g["w"])
    assert np.array_equal(wq, g["wq"]) and np.array_equal(bits16(s), bits16(g["scale"]))
    assert np.array_equal(bits16(of.dequantize_fp8(wq, s)), bits16(g["deq"]))
    assert np.allclose(of.w8a16_ref(g["x"], wq, s), g["y4"], rtol=0, atol=0)


@pytest.mark.gpu
def test_hip_matches_w4a16_fixture():
    from kernels.quant import dequantize, quantize_rtn, unpack_int4
    from kernels.w4a16 import w4a16_matmul

    g = load("w4a16")
    qw, s, z = quantize_rtn(dev(g["w"]), 128)
    assert np.array_equal(to_np(qw), g["qweight"])
    assert np.array_equal(bits16(s), bits16(g["scales"])) and np.array_equal(bits16(z), bits16(g["zeros"]))
    assert np.array_equal(to_np(unpack_int4(qw)), oq.unpack_int4(g["qweight"]))
    assert np.array_equal(bits16(dequantize(qw, s, z)), bits16(g["deq"]))
    assert_north_star(w4a16_matmul(dev(g["x"][:1]), qw, s, z), g["y1"])
    assert_north_star(w4a16_matmul(dev(g["x"]), qw, s, z, bias=dev(g["bias"])), g["y4_bias"])


@pytest.mark.gpu
def test_hip_matches_norm_act_fixture():
    from _util import within_one_ulp_of_intermediate
    from kernels.rmsnorm import rmsnorm
    from kernels.swiglu import swiglu_fused
    from oracle.reference import rmsnorm_parts, silu_ref

    g = load("norm_act")
    out, res = rmsnorm(dev(g["x"]), dev(g["w"]), 1e-6, residual=dev(g["r"]))
    assert np.array_equal(bits16(res), bits16(g["res"]))
    _, normed, _ = rmsnorm_parts(g["x"], g["w"], 1e-6, g["r"])
    assert within_one_ulp_of_intermediate(out, normed, np.broadcast_to(g["w"], normed.shape)).all()
    act = swiglu_fused(dev(g["gate_up"]))
    gu = g["gate_up"]
    assert within_one_ulp_of_intermediate(act, silu_ref(gu[:, :512]), gu[:, 512:]).all()


@pytest.mark.gpu
def test_hip_matches_fp8_fixture():
    from kernels.fp8 import FP8, dequantize_fp8, quantize_fp8, w8a16_matmul

    g = load("fp8")
    wq, s = quantize_fp8(dev(g["w"]))
    assert np.array_equal(to_np(wq.view(torch.uint8)), g["wq"])
    assert np.array_equal(bits16(s), bits16(g["scale"]))
    assert np.array_equal(bits16(dequantize_fp8(wq, s)), bits16(g["deq"]))
    assert_north_star(w8a16_matmul(dev(g["x"]), dev(g["wq"]).view(FP8), dev(g["scale"])), g["y4"])
