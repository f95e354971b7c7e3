"""int4 format kernels vs the oracle, bit for bit: pack/unpack, RTN quantize, dequantize.

unpacked and dequantized weights match the reference bit-exactly."""

import numpy as np
import pytest
import torch

from _util import bits16, dev, to_np
from kernels.bench import cases
from kernels.quant import dequantize, pack_int4, quantize_rtn, unpack_int4, weight_bytes
from oracle import quant as oq
from oracle.reference import dequantize_ref

pytestmark = pytest.mark.gpu


def test_pack_unpack_bit_exact():
    rng = np.random.default_rng(0)
    q = rng.integers(0, 16, (1536, 2048)).astype(np.int32)
    packed = pack_int4(dev(q))
    assert np.array_equal(to_np(packed), oq.pack_int4(q))
    assert np.array_equal(to_np(unpack_int4(packed)), q)


def test_pack_extremes():
    q = torch.full((16, 3), 15, dtype=torch.int32, device="cuda")
    assert torch.equal(pack_int4(q).cpu(), torch.full((2, 3), -1, dtype=torch.int32))


def test_pack_out_of_range_wraps_like_reference():
    """quant.py:24-28 sums q << 4i in int64 and wraps to int32; so does the kernel."""
    rng = np.random.default_rng(1)
    q = rng.integers(-40, 40, (64, 8)).astype(np.int32)
    assert np.array_equal(to_np(pack_int4(dev(q))), oq.pack_int4(q))


@pytest.mark.parametrize("name,N,K", [("gate_up", 17920, 1536), ("down", 1536, 8960),
                                      ("k", 256, 1536)])
def test_quantize_rtn_bit_exact_config_shapes(name, N, K):
    w, _ = cases.w4a16_case(1, N, K, seed=0)
    qw, s, z = quantize_rtn(w.cuda(), 128)
    oqw, os_, oz = oq.quantize_rtn(w.numpy(), 128)
    assert qw.dtype == torch.int32 and s.dtype == torch.float16
    assert np.array_equal(to_np(qw), oqw)
    assert np.array_equal(bits16(s), bits16(os_))
    assert np.array_equal(bits16(z), bits16(oz))


@pytest.mark.parametrize("gs", [32, 64, 256])
def test_quantize_rtn_group_sizes(gs):
    w, _ = cases.w4a16_case(1, 96, 512, seed=5)
    qw, s, z = quantize_rtn(w.cuda(), gs)
    oqw, os_, oz = oq.quantize_rtn(w.numpy(), gs)
    assert np.array_equal(to_np(qw), oqw)
    assert np.array_equal(bits16(s), bits16(os_)) and np.array_equal(bits16(z), bits16(oz))


def test_quantize_rtn_fp32_weight_keeps_fp32_scales():
    w = torch.randn(64, 384, generator=cases.gen(6)) * 0.05
    qw, s, z = quantize_rtn(w.cuda(), 128)
    oqw, os_, oz = oq.quantize_rtn(w.numpy(), 128)
    assert s.dtype == torch.float32
    assert np.array_equal(to_np(qw), oqw)
    assert np.array_equal(to_np(s).view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(to_np(z), oz)


def test_quantize_rtn_bf16_weight():
    """bf16 weights: the oracle runs on the (exact) fp32 values; scales are rounded to bf16 with
    torch's own RNE cast."""
    w = (torch.randn(32, 256, generator=cases.gen(7)) * 0.02).bfloat16()
    qw, s, z = quantize_rtn(w.cuda(), 128)
    oqw, os_, oz = oq.quantize_rtn(w.float().numpy(), 128)
    assert s.dtype == torch.bfloat16
    assert np.array_equal(to_np(qw), oqw)
    assert torch.equal(s.cpu().view(torch.int16), torch.from_numpy(os_).bfloat16().view(torch.int16))
    assert torch.equal(z.cpu().float(), torch.from_numpy(oz))


def test_quantize_rtn_edge_groups():
    """Constant groups (scale clamp), exact grids and ties, with known answers from the oracle
    tests."""
    w = np.zeros((4, 128), dtype=np.float32)
    w[0] = 0.5
    w[1] = -3e-6
    w[2] = (np.arange(128) % 16 - 3) * 0.25
    w[3, 0], w[3, 1] = 0.0, 15.0
    w[3, 2:6] = [2.5, 3.5, 0.5, 14.5]
    qw, s, z = quantize_rtn(dev(w), 128)
    oqw, os_, oz = oq.quantize_rtn(w, 128)
    assert np.array_equal(to_np(qw), oqw)
    assert np.array_equal(to_np(s).view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(to_np(z), oz)


@pytest.mark.parametrize("N,K", [(17920, 1536), (1536, 8960), (40, 384)])
def test_dequantize_bit_exact(N, K):
    w, _ = cases.w4a16_case(1, N, K, seed=0)
    oqw, os_, oz = oq.quantize_rtn(w.numpy(), 128)
    out = dequantize(dev(oqw), dev(os_), dev(oz), 128)
    assert out.shape == (N, K) and out.dtype == torch.float16
    assert np.array_equal(bits16(out), bits16(dequantize_ref(oqw, os_, oz, 128)))


def test_weight_bytes_matches_buffers():
    qw, s, z = quantize_rtn(torch.zeros(17920, 1536, dtype=torch.float16, device="cuda"))
    nbytes = sum(t.numel() * t.element_size() for t in (qw, s, z))
    assert nbytes == weight_bytes(17920, 1536) == 14_622_720


# ------------------------------------------------ CPU tensors in, CPU tensors out (reference
# quant.py:20-49 and fp8.py:25-35 are device-agnostic torch code; its tests call them on the CPU)
def test_cpu_inputs_bit_exact_and_returned_on_cpu():
    from kernels.fp8 import dequantize_fp8, quantize_fp8
    from oracle import fp8 as of

    w, _ = cases.w4a16_case(1, 256, 1536, seed=0)  # fp16 [N, K] on the CPU
    qw, s, z = quantize_rtn(w, 128)
    oqw, os_, oz = oq.quantize_rtn(w.numpy(), 128)
    assert qw.device.type == s.device.type == z.device.type == "cpu"
    assert np.array_equal(qw.numpy(), oqw)
    assert np.array_equal(bits16(s), bits16(os_)) and np.array_equal(bits16(z), bits16(oz))
    deq = dequantize(qw, s, z, 128)
    assert deq.device.type == "cpu"
    assert np.array_equal(bits16(deq), bits16(dequantize_ref(oqw, os_, oz, 128)))
    q = torch.from_numpy(np.random.default_rng(3).integers(0, 16, (64, 40)).astype(np.int32))
    packed = pack_int4(q)
    assert packed.device.type == "cpu" and np.array_equal(packed.numpy(), oq.pack_int4(q.numpy()))
    assert torch.equal(unpack_int4(packed), q)
    wq, sc = quantize_fp8(w)
    owq, osc = of.quantize_fp8(w.numpy())
    assert wq.device.type == sc.device.type == "cpu"
    assert np.array_equal(wq.view(torch.uint8).numpy(), owq) and np.array_equal(bits16(sc), bits16(osc))
    back = dequantize_fp8(wq, sc)
    assert back.device.type == "cpu"
    assert np.array_equal(bits16(back), bits16(of.dequantize_fp8(owq, osc)))


def test_mixed_devices_rejected():
    q = torch.zeros((8, 4), dtype=torch.int32)  # K = 64: one group of 64
    with pytest.raises(RuntimeError, match="different devices"):
        dequantize(q.cuda(), torch.zeros((1, 4), dtype=torch.float16),
                   torch.zeros((1, 4), dtype=torch.float16, device="cuda"), 64)


def test_dequantize_column_sliced_scales_and_zeros():
    """Non-contiguous scales/zeros (column slices of a wider tensor) are copied to temporaries
    that must both stay alive until the launch is enqueued."""
    N, K = 96, 512
    w, _ = cases.w4a16_case(1, 2 * N, K, seed=8)
    oqw, os_, oz = oq.quantize_rtn(w.numpy(), 128)
    qw_t, s_t, z_t = dev(oqw), dev(os_), dev(oz)
    qs, ss, zs = qw_t[:, N:], s_t[:, N:], z_t[:, N:]
    assert not ss.is_contiguous() and not zs.is_contiguous()
    out = dequantize(qs, ss, zs, 128)
    ref = dequantize_ref(np.ascontiguousarray(oqw[:, N:]), np.ascontiguousarray(os_[:, N:]),
                         np.ascontiguousarray(oz[:, N:]), 128)
    assert np.array_equal(bits16(out), bits16(ref))
