"""The PyTorch-CPU restatement (oracle/torch_cpu.py, the CPU baseline that bench.py times) against
the pinned numpy oracle on the same seeded inputs: dequantized weights and the RMSNorm residual bit
for bit, RMSNorm and SwiGLU within one fp16 step, the fp32 matmuls within reduction-order
tolerance of float64, plus the reference's known answer for
unpacking (all-15 nibbles pack to -1, tests/test_quant.py:15-18)."""

import numpy as np
import torch

from kernels.bench import cases
from oracle import fp8 as of
from oracle import quant as oq
from oracle import reference as ref
from oracle import torch_cpu as tc


def _bits(t):
    return t.numpy().view(np.uint16)


def test_unpack_known_answer_and_round_trip():
    assert torch.equal(tc.unpack_int4(torch.full((1, 3), -1, dtype=torch.int32)),
                       torch.full((8, 3), 15, dtype=torch.int32))
    q = np.random.default_rng(0).integers(0, 16, (64, 24)).astype(np.int32)
    assert np.array_equal(tc.unpack_int4(torch.from_numpy(oq.pack_int4(q))).numpy(), q)


def test_dequantize_and_matmul_match_numpy_oracle():
    w, x = cases.w4a16_case(3, 256, 1536, seed=0)
    qw, s, z = oq.quantize_rtn(w.numpy(), 128)
    t = tuple(torch.from_numpy(a) for a in (qw, s, z))
    assert np.array_equal(_bits(tc.dequantize_ref(*t)), ref.dequantize_ref(qw, s, z).view(np.uint16))
    y = tc.w4a16_ref(x, *t).numpy()
    y64 = ref.w4a16_ref_f64(x.numpy(), qw, s, z)
    assert np.abs(y - y64).max() <= 1e-4 * max(1.0, np.abs(y64).max())


def test_rmsnorm_and_swiglu_bit_exact():
    xr, r, wr = cases.rmsnorm_case(16, 1536, seed=1)
    out, res = tc.rmsnorm_ref(xr, wr, 1e-6, residual=r)
    oo, orr = ref.rmsnorm_ref(xr.numpy(), wr.numpy(), 1e-6, residual=r.numpy())
    assert np.array_equal(_bits(res), orr.view(np.uint16))
    # the mean of squares may be reduced in another order: at most one fp16 step apart
    d = np.abs(out.float().numpy() - oo.astype(np.float32))
    assert (d <= 2.0 ** -10 * np.maximum(np.abs(oo.astype(np.float32)), 2.0 ** -14) * 2).all()
    gu = cases.swiglu_case(16, 8960, seed=1)
    a = tc.swiglu_ref(gu[:, :8960], gu[:, 8960:])
    b = ref.swiglu_ref(gu[:, :8960].numpy(), gu[:, 8960:].numpy())
    assert (np.abs(a.float().numpy() - b.astype(np.float32)) <= 2e-3 * np.abs(b.astype(np.float32)) + 1e-3).all()


def test_fp8_dequantize_and_matmul_match_numpy_oracle():
    w, x = cases.w4a16_case(2, 128, 512, seed=3)
    wq, sc = of.quantize_fp8(w.numpy())
    wq_t = torch.from_numpy(wq).view(torch.float8_e4m3fn)
    deq = tc.dequantize_fp8(wq_t, torch.from_numpy(sc))
    assert np.array_equal(_bits(deq), of.dequantize_fp8(wq, sc).view(np.uint16))
    y = tc.w8a16_ref(x, wq_t, torch.from_numpy(sc)).numpy()
    y64 = x.numpy().astype(np.float64) @ of.dequantize_fp8(wq, sc).astype(np.float64).T
    assert np.abs(y - y64).max() <= 1e-4 * max(1.0, np.abs(y64).max())
