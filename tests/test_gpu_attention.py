"""The fused decode attention kernel (ldk_decode_attention) against a float64 CPU computation of
the same block: RoPE with exact cos/sin (rotate_half pairing, kernels/e2e/model.py:212-214 of the
reference), the cache write at pos, and grouped-query softmax attention over positions 0..pos
(model.py:236-243)."""

import math

import numpy as np
import pytest
import torch

from kernels.attention import decode_attention

pytestmark = pytest.mark.gpu


def _rope64(x, pos, inv_freq):
    """float64 RoPE of x [..., 128] at position pos (angles from the fp32 inv_freq values)."""
    ang = float(pos) * inv_freq.astype(np.float64)
    ang = np.concatenate([ang, ang])
    rh = np.concatenate([-x[..., 64:], x[..., :64]], axis=-1)
    return x * np.cos(ang) + rh * np.sin(ang)


@pytest.mark.parametrize("nq,nkv,L,pos", [(12, 2, 392, 0), (12, 2, 392, 127), (12, 2, 392, 383),
                                          (12, 2, 392, 391), (12, 2, 392, 320), (4, 4, 64, 63),
                                          (8, 1, 512, 511), (16, 2, 136, 64), (12, 2, 8, 5),
                                          (12, 2, 2048, 1500), (12, 2, 4096, 4095),
                                          (72, 8, 256, 200), (64, 8, 2048, 2047),
                                          (12, 2, 2112, 2111), (12, 2, 40000, 39999),
                                          (12, 2, 40000, 700)])
def test_against_float64(nq, nkv, L, pos):
    """Cache lengths cover one position range (up to 512 positions), several ranges of 8 chunks
    with a short last one (2048, 2112: 4 and 5 ranges, 4096: 8), 32 ranges of 20 chunks with
    8 waves looping (40000), pos in the first range of a split cache (40000, 700), and more
    heads than can split (72)."""
    g = torch.Generator().manual_seed(pos + 7 * nq)
    hd = 128
    qkv = torch.randn((nq + 2 * nkv) * hd, generator=g).half()
    kt = (torch.randn(1, nkv, hd, L, generator=g) * 0.7).half()
    vc = torch.randn(1, nkv, L, hd, generator=g).half()
    inv_freq = (1.0 / (1e6 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd)))
    kt_d, vc_d = kt.cuda(), vc.cuda()
    out = decode_attention(qkv.cuda().view(1, 1, -1), torch.tensor([pos], device="cuda"),
                           inv_freq.cuda(), kt_d, vc_d, nq, nkv, hd ** -0.5)
    x = qkv.double().numpy()
    q = x[: nq * hd].reshape(nq, hd)
    k = x[nq * hd:(nq + nkv) * hd].reshape(nkv, hd)
    v = x[(nq + nkv) * hd:].reshape(nkv, hd)
    fr = inv_freq.numpy()
    qr, kr = _rope64(q, pos, fr), _rope64(k, pos, fr)
    # the cache now holds the new k (roped) and v at pos, untouched elsewhere
    kt_got, vc_got = kt_d.cpu().double().numpy(), vc_d.cpu().double().numpy()
    assert np.abs(kt_got[0, :, :, pos] - kr).max() <= 4e-3 * max(1.0, np.abs(kr).max())
    assert np.array_equal(vc_got[0, :, pos], v.astype(np.float16).astype(np.float64))
    mask = np.ones(L, dtype=bool)
    mask[pos] = False
    assert np.array_equal(kt_got[0][..., mask], kt.double().numpy()[0][..., mask])
    assert np.array_equal(vc_got[0][:, mask], vc.double().numpy()[0][:, mask])
    # attention in float64 over positions 0..pos with the new k/v (as stored in fp16)
    K = kt_got[0].transpose(0, 2, 1)[:, : pos + 1]  # [nkv, pos+1, hd]
    V = vc_got[0][:, : pos + 1]
    gq = nq // nkv
    ref = np.zeros((nq, hd))
    for h in range(nq):
        s = K[h // gq] @ qr[h] / math.sqrt(hd)
        p = np.exp(s - s.max())
        ref[h] = (p / p.sum()) @ V[h // gq]
    got = out.view(nq, hd).cpu().double().numpy()
    err = np.abs(got - ref)
    assert err.max() <= 2e-2 and np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 2e-3, (err.max(),)


def test_rejects_unsupported_shapes():
    qkv = torch.zeros(16 * 128, dtype=torch.float16, device="cuda")
    kt = torch.zeros(1, 2, 128, 602, dtype=torch.float16, device="cuda")
    vc = torch.zeros(1, 2, 602, 128, dtype=torch.float16, device="cuda")
    inv = torch.ones(64, device="cuda")
    with pytest.raises(RuntimeError):  # max_len 602 is not a multiple of 8
        decode_attention(qkv, torch.tensor([0], device="cuda"), inv, kt, vc, 12, 2, 1.0)


def test_pos_past_the_cache_writes_nothing():
    """pos >= max_len: attention over the whole cache, the cache is left as it was."""
    nq, nkv, L, hd = 12, 2, 64, 128
    g = torch.Generator().manual_seed(3)
    qkv = torch.randn((nq + 2 * nkv) * hd, generator=g).half().cuda()
    kt = (torch.randn(1, nkv, hd, L, generator=g) * 0.7).half().cuda()
    vc = torch.randn(1, nkv, L, hd, generator=g).half().cuda()
    kt0, vc0 = kt.clone(), vc.clone()
    inv = torch.ones(64, device="cuda")
    out = decode_attention(qkv, torch.tensor([L], device="cuda"), inv, kt, vc, nq, nkv, hd ** -0.5)
    assert torch.equal(kt, kt0) and torch.equal(vc, vc0)
    assert torch.isfinite(out).all()


def _reference(qkv, kt_now, vc_now, nq, nkv, pos, inv_freq):
    hd = 128
    x = qkv.double().cpu().numpy()
    q = _rope64(x[: nq * hd].reshape(nq, hd), pos, inv_freq.cpu().numpy())
    K = kt_now[0].transpose(0, 2, 1)[:, : pos + 1]
    V = vc_now[0][:, : pos + 1]
    gq = nq // nkv
    ref = np.zeros((nq, hd))
    for h in range(nq):
        s = K[h // gq] @ q[h] / math.sqrt(hd)
        p = np.exp(s - s.max())
        ref[h] = (p / p.sum()) @ V[h // gq]
    return ref


@pytest.mark.parametrize("L,steps", [(512, 301), (1536, 1100)])
def test_decode_sequence_two_layers(L, steps):
    """Decode steps over two layers' caches, as the runner issues them: every step writes its
    k/v and attends over 0..pos. A 1536-position cache has three 512-position ranges, so from
    pos 512 on a head's ranges meet through the shared partials and arrival counters, which each
    launch must leave zeroed for the next."""
    nq, nkv, hd = 12, 2, 128
    g = torch.Generator().manual_seed(11)
    inv = (1.0 / (1e6 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))).cuda()
    caches = [((torch.randn(1, nkv, hd, L, generator=g) * 0.7).half().cuda(),
               torch.randn(1, nkv, L, hd, generator=g).half().cuda()) for _ in range(2)]
    pos_t = torch.zeros(1, dtype=torch.int64, device="cuda")
    edges = (63, 64, 65, 127, 128, 511, 512, 513, 1023, 1024, 1025, steps - 1)
    for pos in range(steps):
        pos_t.fill_(pos)
        for li, (kt, vc) in enumerate(caches):
            qkv = torch.randn((nq + 2 * nkv) * hd, generator=g).half().cuda()
            out = decode_attention(qkv, pos_t, inv, kt, vc, nq, nkv, hd ** -0.5)
            if pos % 50 == 0 or pos in edges:
                ref = _reference(qkv, kt.cpu().double().numpy(), vc.cpu().double().numpy(), nq, nkv,
                                 pos, inv)
                got = out.view(nq, hd).cpu().double().numpy()
                assert np.abs(got - ref).max() <= 2e-2, (pos, li)
                assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 2e-3, (pos, li)


def test_negative_pos_attends_nothing():
    """pos < 0: no live position, the output is zero and the cache is left as it was."""
    nq, nkv, L, hd = 12, 2, 256, 128
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn((nq + 2 * nkv) * hd, generator=g).half().cuda()
    kt = torch.randn(1, nkv, hd, L, generator=g).half().cuda()
    vc = torch.randn(1, nkv, L, hd, generator=g).half().cuda()
    kt0, vc0 = kt.clone(), vc.clone()
    out = decode_attention(qkv, torch.tensor([-1], device="cuda"), torch.ones(64, device="cuda"),
                           kt, vc, nq, nkv, hd ** -0.5)
    assert torch.equal(kt, kt0) and torch.equal(vc, vc0)
    assert torch.count_nonzero(out) == 0
