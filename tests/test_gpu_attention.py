"""The fused decode attention kernel (ldk_decode_attention) against a float64 CPU computation of
the same block: RoPE with exact cos/sin (rotate_half pairing, kernels/e2e/model.py:212-214 of the
reference), the cache write at pos, and grouped-query softmax attention over positions 0..pos
(model.py:236-243)."""

import math

import numpy as np
import pytest
import torch

from kernels.attention import decode_attention, k_from_tiles, k_to_tiles, v_from_tiles, vt_to_tiles

pytestmark = pytest.mark.gpu


def _rope64(x, pos, inv_freq):
    """float64 RoPE of x [..., 128] at position pos (angles from the fp32 inv_freq values)."""
    ang = float(pos) * inv_freq.astype(np.float64)
    ang = np.concatenate([ang, ang])
    rh = np.concatenate([-x[..., 64:], x[..., :64]], axis=-1)
    return x * np.cos(ang) + rh * np.sin(ang)


def _caches(g, nkv, L, hd=128):
    """Random K and V [1, nkv, L, hd] fp16 and their tiled device caches."""
    kc = (torch.randn(1, nkv, L, hd, generator=g) * 0.7).half()
    vc = torch.randn(1, nkv, L, hd, generator=g).half()
    return kc, vc, k_to_tiles(kc).cuda(), vt_to_tiles(vc).cuda()


@pytest.mark.parametrize("nq,nkv,L,pos", [(12, 2, 416, 0), (12, 2, 416, 127), (12, 2, 416, 383),
                                          (12, 2, 416, 415), (12, 2, 416, 320), (4, 4, 64, 63),
                                          (8, 1, 512, 511), (16, 2, 160, 64), (12, 2, 32, 5),
                                          (12, 2, 2048, 1500), (12, 2, 4096, 4095),
                                          (72, 8, 256, 200), (64, 8, 2048, 2047),
                                          (12, 2, 2144, 2143), (12, 2, 40000, 39999),
                                          (12, 2, 40000, 700), (40, 2, 288, 200),
                                          (36, 1, 1056, 1055), (16, 1, 384, 383),
                                          (144, 8, 1536, 1100), (14, 2, 8192, 6000)])
def test_against_float64(nq, nkv, L, pos):
    """Cache lengths cover one position range (up to 512 positions) with pos at chunk edges,
    128-position ranges with a short last one (2048: 16, 2144: 17; 4096: 32), 32 ranges of
    1280 positions that each wave takes in three passes (40000), pos in the first range of a
    split cache (40000, 700), more query heads per kv head than one 16-head tile (40/2: two
    tiles, 36/1: three tiles over nine ranges), a full tile (16/1), seven heads per kv head
    (14/2), and more heads than the range partials hold (72 heads in one range; 144 heads: one
    range of 1536 positions per tile)."""
    g = torch.Generator().manual_seed(pos + 7 * nq)
    hd = 128
    qkv = torch.randn((nq + 2 * nkv) * hd, generator=g).half()
    kc, vc, kt_d, vt_d = _caches(g, nkv, L)
    inv_freq = (1.0 / (1e6 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd)))
    out = decode_attention(qkv.cuda().view(1, 1, -1), torch.tensor([pos], device="cuda"),
                           inv_freq.cuda(), kt_d, vt_d, nq, nkv, hd ** -0.5)
    x = qkv.double().numpy()
    q = x[: nq * hd].reshape(nq, hd)
    k = x[nq * hd:(nq + nkv) * hd].reshape(nkv, hd)
    v = x[(nq + nkv) * hd:].reshape(nkv, hd)
    fr = inv_freq.numpy()
    qr, kr = _rope64(q, pos, fr), _rope64(k, pos, fr)
    # the cache now holds the new k (roped) and v at pos, untouched elsewhere
    k_got = k_from_tiles(kt_d.cpu()).double().numpy()
    v_got = v_from_tiles(vt_d.cpu()).double().numpy()
    assert np.abs(k_got[0, :, pos] - kr).max() <= 4e-3 * max(1.0, np.abs(kr).max())
    assert np.array_equal(v_got[0, :, pos], v.astype(np.float16).astype(np.float64))
    mask = np.ones(L, dtype=bool)
    mask[pos] = False
    assert np.array_equal(k_got[0][:, mask], kc.double().numpy()[0][:, mask])
    assert np.array_equal(v_got[0][:, mask], vc.double().numpy()[0][:, mask])
    # attention in float64 over positions 0..pos with the new k/v (as stored in fp16)
    K = k_got[0][:, : pos + 1]  # [nkv, pos+1, hd]
    V = v_got[0][:, : pos + 1]
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
    inv = torch.ones(64, device="cuda")
    kc = torch.zeros(1, 2, 1, 2, 4, 16, 32, dtype=torch.float16, device="cuda")
    vt = torch.zeros(1, 2, 1, 8, 16, 32, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError):  # head_dim 64
        from kernels import _lib

        st = _lib.load().ldk_decode_attention(
            _lib.ptr(qkv), _lib.ptr(torch.zeros(1, dtype=torch.int64, device="cuda")), _lib.ptr(inv),
            _lib.ptr(kc), _lib.ptr(vt), _lib.ptr(qkv), 12, 2, 64, 32, 1.0, None, None, 0,
            _lib.stream(qkv.device))
        _lib.check(st, "decode_attention")
    with pytest.raises(RuntimeError):  # max_len 40 is not a multiple of 32
        st = _lib.load().ldk_decode_attention(
            _lib.ptr(qkv), _lib.ptr(torch.zeros(1, dtype=torch.int64, device="cuda")), _lib.ptr(inv),
            _lib.ptr(kc), _lib.ptr(vt), _lib.ptr(qkv), 12, 2, 128, 40, 1.0, None, None, 0,
            _lib.stream(qkv.device))
        _lib.check(st, "decode_attention")


def test_pos_past_the_cache_writes_nothing():
    """pos >= max_len: attention over the whole cache, the cache is left as it was."""
    nq, nkv, L, hd = 12, 2, 64, 128
    g = torch.Generator().manual_seed(3)
    qkv = torch.randn((nq + 2 * nkv) * hd, generator=g).half().cuda()
    _, _, kc, vt = _caches(g, nkv, L)
    kc0, vt0 = kc.clone(), vt.clone()
    inv = torch.ones(64, device="cuda")
    out = decode_attention(qkv, torch.tensor([L], device="cuda"), inv, kc, vt, nq, nkv, hd ** -0.5)
    assert torch.equal(kc, kc0) and torch.equal(vt, vt0)
    assert torch.isfinite(out).all()


def _reference(qkv, k_tiles, vt_tiles, nq, nkv, pos, inv_freq):
    hd = 128
    x = qkv.double().cpu().numpy()
    q = _rope64(x[: nq * hd].reshape(nq, hd), pos, inv_freq.cpu().numpy())
    K = k_from_tiles(k_tiles.cpu()).double().numpy()[0][:, : pos + 1]
    V = v_from_tiles(vt_tiles.cpu()).double().numpy()[0][:, : pos + 1]
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
    k/v and attends over 0..pos. A 1536-position cache has twelve 128-position ranges, so from
    pos 128 on a head's ranges meet through the shared partials in the merge launch, which must
    skip the stale partials of ranges that earlier steps left behind."""
    nq, nkv, hd = 12, 2, 128
    g = torch.Generator().manual_seed(11)
    inv = (1.0 / (1e6 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))).cuda()
    caches = [_caches(g, nkv, L)[2:] for _ in range(2)]
    pos_t = torch.zeros(1, dtype=torch.int64, device="cuda")
    edges = (63, 64, 65, 127, 128, 129, 255, 256, 511, 512, 513, 1023, 1024, 1025, steps - 1)
    for pos in range(steps):
        pos_t.fill_(pos)
        for li, (kc, vt) in enumerate(caches):
            qkv = torch.randn((nq + 2 * nkv) * hd, generator=g).half().cuda()
            out = decode_attention(qkv, pos_t, inv, kc, vt, nq, nkv, hd ** -0.5)
            if pos % 50 == 0 or pos in edges:
                ref = _reference(qkv, kc, vt, nq, nkv, pos, inv)
                got = out.view(nq, hd).cpu().double().numpy()
                assert np.abs(got - ref).max() <= 2e-2, (pos, li)
                assert np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 2e-3, (pos, li)


def test_negative_pos_attends_nothing():
    """pos < 0: no live position, the output is zero and the cache is left as it was."""
    nq, nkv, L, hd = 12, 2, 256, 128
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn((nq + 2 * nkv) * hd, generator=g).half().cuda()
    _, _, kc, vt = _caches(g, nkv, L)
    kc0, vt0 = kc.clone(), vt.clone()
    out = decode_attention(qkv, torch.tensor([-1], device="cuda"), torch.ones(64, device="cuda"),
                           kc, vt, nq, nkv, hd ** -0.5)
    assert torch.equal(kc, kc0) and torch.equal(vt, vt0)
    assert torch.count_nonzero(out) == 0


def _w4_linear(g, N, K):
    from kernels.quant import quantize_rtn

    w = (torch.randn(N, K, generator=g) * 0.02).half()
    qw, s, z = quantize_rtn(w.cuda(), 128)
    return qw, s, z


@pytest.mark.parametrize("L,pos", [(416, 0), (416, 31), (416, 127), (416, 128), (416, 200),
                                   (416, 383), (416, 384), (416, 415), (416, 700), (416, -3),
                                   (256, 255), (128, 77), (32, 5)])
def test_ranges_merged_in_o_projection(L, pos):
    """decode_attention_ranges + attn_linear_rmsnorm_w4a16_matmul (the attention's ranges merged
    in the o projection's x staging) against decode_attention + linear_rmsnorm_w4a16_matmul on the
    same inputs: pos in each of the four ranges of 416 positions (128 each, the last one 32) and
    at their edges, past the cache (the whole cache, no write) and negative (no position: zeros),
    and shorter caches (256: ranges of 64; 128: 32; 32: one range). The cache updates are
    bit-identical; y and the residual stream h agree to the north-star bound (the merged x can
    differ from the merge launch's in the last fp16 bit)."""
    from _util import assert_north_star
    from kernels.attention import decode_attention_ranges, ranges_len
    from kernels.fused import attn_linear_rmsnorm_w4a16_matmul, linear_rmsnorm_w4a16_matmul

    nq, nkv, hd, H, I2 = 12, 2, 128, 1536, 2 * 1024
    g = torch.Generator().manual_seed(1000 + L + pos)
    qkv = torch.randn((nq + 2 * nkv) * hd, generator=g).half().cuda().view(1, 1, -1)
    _, _, kt_a, vt_a = _caches(g, nkv, L)
    kt_b, vt_b = kt_a.clone(), vt_a.clone()
    inv_freq = (1.0 / (1e6 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))).cuda()
    p = torch.tensor([pos], device="cuda")
    qo, so, zo = _w4_linear(g, H, nq * hd)
    qg, sg, zg = _w4_linear(g, I2, H)
    bo = (torch.randn(H, generator=g) * 0.1).half().cuda()
    res = torch.randn(1, 1, H, generator=g).half().cuda()
    nw = (1 + 0.1 * torch.randn(H, generator=g)).half().cuda()

    attn = decode_attention(qkv, p, inv_freq, kt_a, vt_a, nq, nkv, hd ** -0.5)
    y_ref, h_ref = linear_rmsnorm_w4a16_matmul(attn, qo, so, zo, bo, res, nw, 1e-6, qg, sg, zg)
    rng = decode_attention_ranges(qkv, p, inv_freq, kt_b, vt_b, nq, nkv, hd ** -0.5, ranges_len(L))
    y, h = attn_linear_rmsnorm_w4a16_matmul(rng, qo, so, zo, bo, res, nw, 1e-6, qg, sg, zg)
    assert torch.equal(kt_a, kt_b) and torch.equal(vt_a, vt_b)
    for got, ref in ((h, h_ref), (y, y_ref)):
        assert torch.isfinite(got).all()
        assert_north_star(got.cpu(), ref.float().cpu().numpy())
        d = (got.float() - ref.float()).abs()
        assert (d <= 2e-3 * ref.float().abs() + 2e-3).float().mean() >= 0.999


@pytest.mark.parametrize("L,pos", [(416, 0), (416, 127), (416, 128), (416, 300), (416, 415),
                                   (416, 700), (416, -3), (256, 255), (32, 5)])
def test_ranges_merged_in_fp8_o_projection(L, pos):
    """decode_attention_ranges + attn_w8a16_matmul (the ranges merged in the e4m3 o projection's
    x staging) against decode_attention + w8a16_matmul on the same inputs, with bias: pos in and
    at the edges of the four ranges of 416 positions, past the cache, negative (zeros), shorter
    caches. The cache updates are bit-identical; y agrees to the north-star bound (the merged x
    can differ from the merge launch's in the last fp16 bit)."""
    from _util import assert_north_star
    from kernels.attention import decode_attention_ranges, ranges_len
    from kernels.fp8 import quantize_fp8, w8a16_matmul
    from kernels.fused import attn_w8a16_matmul

    nq, nkv, hd, H = 12, 2, 128, 1536
    g = torch.Generator().manual_seed(2000 + L + pos)
    qkv = torch.randn((nq + 2 * nkv) * hd, generator=g).half().cuda().view(1, 1, -1)
    _, _, kt_a, vt_a = _caches(g, nkv, L)
    kt_b, vt_b = kt_a.clone(), vt_a.clone()
    inv_freq = (1.0 / (1e6 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))).cuda()
    p = torch.tensor([pos], device="cuda")
    wq, sc = quantize_fp8((torch.randn(H, nq * hd, generator=g) * 0.02).half().cuda())
    bo = (torch.randn(H, generator=g) * 0.1).half().cuda()

    attn = decode_attention(qkv, p, inv_freq, kt_a, vt_a, nq, nkv, hd ** -0.5)
    y_ref = w8a16_matmul(attn.view(1, -1), wq, sc, bias=bo)
    rng = decode_attention_ranges(qkv, p, inv_freq, kt_b, vt_b, nq, nkv, hd ** -0.5, ranges_len(L))
    y = attn_w8a16_matmul(rng, wq, sc, bo)
    assert torch.equal(kt_a, kt_b) and torch.equal(vt_a, vt_b)
    assert torch.isfinite(y).all() and y.shape == (1, H)
    assert_north_star(y.cpu(), y_ref.float().cpu().numpy())
    d = (y.float() - y_ref.float()).abs()
    assert (d <= 2e-3 * y_ref.float().abs() + 2e-3).float().mean() >= 0.999


def test_fp8_ranges_consumer_checks_stream_and_geometry():
    """The e4m3 o projection that merges the ranges is refused on another stream, with another
    range length, or after decode_attention's own range launch overwrote the partials; the
    attention's stream works; more than four ranges is refused before any launch."""
    from kernels import _lib
    from kernels.attention import decode_attention_ranges, ranges_len
    from kernels.fp8 import quantize_fp8
    from kernels.fused import attn_w8a16_matmul

    nq, nkv, hd, H, L = 12, 2, 128, 1536, 416
    g = torch.Generator().manual_seed(79)
    qkv = torch.randn((nq + 2 * nkv) * hd, generator=g).half().cuda().view(1, 1, -1)
    _, _, kt, vt = _caches(g, nkv, L)
    inv_freq = (1.0 / (1e6 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))).cuda()
    wq, sc = quantize_fp8((torch.randn(H, nq * hd, generator=g) * 0.02).half().cuda())
    p = torch.tensor([300], device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        rng = decode_attention_ranges(qkv, p, inv_freq, kt, vt, nq, nkv, hd ** -0.5, ranges_len(L))
    torch.cuda.synchronize()
    with pytest.raises(ValueError, match="another stream"):
        attn_w8a16_matmul(rng, wq, sc)
    with torch.cuda.stream(side):
        y = attn_w8a16_matmul(rng, wq, sc)
        with pytest.raises(ValueError, match="rlen"):
            attn_w8a16_matmul(rng._replace(rlen=L), wq, sc)
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    _, _, kt2, vt2 = _caches(g, nkv, 1024)
    decode_attention(qkv, torch.tensor([900], device="cuda"), inv_freq, kt2, vt2, nq, nkv, hd ** -0.5)
    with pytest.raises(ValueError, match="pending"):
        attn_w8a16_matmul(rng, wq, sc)
    lib = _lib.load()
    st = lib.ldk_w8a16_attn_matmul(_lib.ptr(p), 416, 64, 12, _lib.ptr(wq), _lib.ptr(sc), None,
                                   _lib.ptr(wq), H, nq * hd, None, 0, None)
    assert st == _lib.ERR_UNSUPPORTED


def test_ranges_entry_rejects_bad_ranges():
    """More than the four ranges the o projection merges, or a range length that is not a
    multiple of 32, is refused before any launch."""
    from kernels import _lib

    lib = _lib.load()
    p = torch.zeros(1, dtype=torch.long, device="cuda")
    dummy = torch.zeros(16, dtype=torch.int32, device="cuda")
    st = lib.ldk_w4a16_attn_matmul_residual_stats(
        _lib.ptr(p), 416, 64, 12, _lib.ptr(dummy), _lib.ptr(dummy), _lib.ptr(dummy),
        _lib.ptr(dummy), _lib.ptr(dummy), _lib.ptr(dummy), None, 1536, 1536, 128, None, 0, None)
    assert st == _lib.ERR_UNSUPPORTED
    st = lib.ldk_decode_attention_ranges(_lib.ptr(dummy), _lib.ptr(p), _lib.ptr(dummy),
                                         _lib.ptr(dummy), _lib.ptr(dummy), 12, 2, 128, 416, 100,
                                         0.1, None, None, 0, None)
    assert st == _lib.ERR_UNSUPPORTED


def test_ranges_warm_changes_nothing():
    """The attention launch that also reads byte ranges into the caches (decode_attention_ranges'
    warm tensors: the o and gate_up weights, a 40 MB buffer that takes several passes of the
    warming workgroups, ranges of 16 bytes and of odd 16-byte multiples, an empty tensor) leaves
    the cache update and the merged o projection bit-identical to the launch without them."""
    from kernels.attention import decode_attention_ranges, ranges_len
    from kernels.fused import attn_linear_rmsnorm_w4a16_matmul

    nq, nkv, hd, H, I2, L = 12, 2, 128, 1536, 2 * 1024, 416
    g = torch.Generator().manual_seed(77)
    qkv = torch.randn((nq + 2 * nkv) * hd, generator=g).half().cuda().view(1, 1, -1)
    _, _, kt_a, vt_a = _caches(g, nkv, L)
    kt_b, vt_b = kt_a.clone(), vt_a.clone()
    inv_freq = (1.0 / (1e6 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))).cuda()
    qo, so, zo = _w4_linear(g, H, nq * hd)
    qg, sg, zg = _w4_linear(g, I2, H)
    res = torch.randn(1, 1, H, generator=g).half().cuda()
    nw = (1 + 0.1 * torch.randn(H, generator=g)).half().cuda()
    big = torch.randint(0, 1 << 30, (10 << 20,), dtype=torch.int32, generator=g).cuda()
    odd = torch.zeros(16 * 37 + 16 * 4099, dtype=torch.uint8, device="cuda")
    warm = [qo, qg, sg, zg, big, odd[:16], odd[16 * 37:], torch.empty(0, device="cuda")]
    for pos in (0, 200, 415):
        p = torch.tensor([pos], device="cuda")
        outs = []
        for kt, vt, w in ((kt_a, vt_a, ()), (kt_b, vt_b, warm)):
            rng = decode_attention_ranges(qkv, p, inv_freq, kt, vt, nq, nkv, hd ** -0.5,
                                          ranges_len(L), warm=w)
            outs.append(attn_linear_rmsnorm_w4a16_matmul(rng, qo, so, zo, None, res, nw, 1e-6,
                                                         qg, sg, zg))
        assert torch.equal(kt_a, kt_b) and torch.equal(vt_a, vt_b)
        assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


def test_ranges_warm_rejects_bad_ranges():
    """Warm ranges are checked before any launch: more than 8, a null array, a pointer that is
    not 16-byte aligned and a size that is not a multiple of 16 are refused."""
    import ctypes

    from kernels import _lib

    lib = _lib.load()
    p = torch.zeros(1, dtype=torch.long, device="cuda")
    buf = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    qkv = torch.zeros(16 * 128, dtype=torch.float16, device="cuda")
    kt = torch.zeros(2 * 32 * 128, dtype=torch.float16, device="cuda")
    freq = torch.zeros(64, dtype=torch.float32, device="cuda")

    def call(ptrs, sizes, n, arrays=True):
        wp = (ctypes.c_void_p * 9)(*ptrs) if arrays else None
        wb = (ctypes.c_int64 * 9)(*sizes) if arrays else None
        return lib.ldk_decode_attention_ranges(_lib.ptr(qkv), _lib.ptr(p), _lib.ptr(freq),
                                               _lib.ptr(kt), _lib.ptr(kt), 12, 2, 128, 32, 32,
                                               0.1, wp, wb, n, None)

    base = buf.data_ptr()
    assert call([base] * 9, [16] * 9, 9) == _lib.ERR_INVALID
    assert call([], [], 1, arrays=False) == _lib.ERR_INVALID
    assert call([base + 8], [16], 1) == _lib.ERR_ALIGN
    assert call([base], [24], 1) == _lib.ERR_ALIGN
    assert call([base], [-16], 1) == _lib.ERR_ALIGN


def test_ranges_consumer_checks_stream_and_geometry():
    """The o projection that merges the attention's ranges reads library-owned partials, so it is
    refused unless the last decode_attention_ranges call on the device left them on its stream
    with its geometry: another stream, another range length, and partials overwritten by
    decode_attention's own range launch (a cache of more than 512 positions) are errors; the same
    stream works."""
    from kernels.attention import decode_attention_ranges, ranges_len
    from kernels.fused import attn_linear_rmsnorm_w4a16_matmul

    nq, nkv, hd, H, I2, L = 12, 2, 128, 1536, 2 * 1024, 416
    g = torch.Generator().manual_seed(78)
    qkv = torch.randn((nq + 2 * nkv) * hd, generator=g).half().cuda().view(1, 1, -1)
    _, _, kt, vt = _caches(g, nkv, L)
    inv_freq = (1.0 / (1e6 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))).cuda()
    qo, so, zo = _w4_linear(g, H, nq * hd)
    qg, sg, zg = _w4_linear(g, I2, H)
    res = torch.randn(1, 1, H, generator=g).half().cuda()
    nw = (1 + 0.1 * torch.randn(H, generator=g)).half().cuda()
    p = torch.tensor([300], device="cuda")

    def merge(rng):
        return attn_linear_rmsnorm_w4a16_matmul(rng, qo, so, zo, None, res, nw, 1e-6, qg, sg, zg)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        rng = decode_attention_ranges(qkv, p, inv_freq, kt, vt, nq, nkv, hd ** -0.5, ranges_len(L))
    torch.cuda.synchronize()
    with pytest.raises(ValueError, match="another stream"):
        merge(rng)
    with torch.cuda.stream(side):
        y, _ = merge(rng)
        with pytest.raises(ValueError, match="rlen"):
            merge(rng._replace(rlen=L))
    torch.cuda.synchronize()
    assert torch.isfinite(y).all()
    _, _, kt2, vt2 = _caches(g, nkv, 1024)
    decode_attention(qkv, torch.tensor([900], device="cuda"), inv_freq, kt2, vt2, nq, nkv, hd ** -0.5)
    with pytest.raises(ValueError, match="pending"):
        merge(rng)


@pytest.mark.parametrize("L,pos", [(416, 300), (1024, 900), (4096, 4000)])
def test_decode_attention_warm_changes_nothing(L, pos):
    """decode_attention with warm tensors (one range, and several ranges with their merge
    launch) returns the same output and cache update, bit for bit, as without them."""
    nq, nkv, hd = 12, 2, 128
    g = torch.Generator().manual_seed(79 + L)
    qkv = torch.randn((nq + 2 * nkv) * hd, generator=g).half().cuda().view(1, 1, -1)
    _, _, kt_a, vt_a = _caches(g, nkv, L)
    kt_b, vt_b = kt_a.clone(), vt_a.clone()
    inv_freq = (1.0 / (1e6 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))).cuda()
    warm = [torch.randint(0, 1 << 30, (3 << 20,), dtype=torch.int32, generator=g).cuda(),
            torch.zeros(4096, dtype=torch.uint8, device="cuda")]
    p = torch.tensor([pos], device="cuda")
    a = decode_attention(qkv, p, inv_freq, kt_a, vt_a, nq, nkv, hd ** -0.5)
    b = decode_attention(qkv, p, inv_freq, kt_b, vt_b, nq, nkv, hd ** -0.5, warm=warm)
    assert torch.equal(a, b) and torch.equal(kt_a, kt_b) and torch.equal(vt_a, vt_b)


@pytest.mark.parametrize("nq,nkv,L,p0,T", [(12, 2, 416, 0, 128), (12, 2, 416, 0, 1), (12, 2, 416, 0, 17),
                                           (12, 2, 416, 100, 60), (12, 2, 416, 380, 36),
                                           (4, 4, 64, 0, 64), (8, 1, 512, 0, 300), (16, 2, 160, 33, 7),
                                           (12, 2, 2048, 0, 1000), (40, 2, 288, 5, 90)])
def test_prefill_against_float64(nq, nkv, L, p0, T):
    """ldk_prefill_attention: T prompt tokens at positions p0 .. p0 + T - 1 over a cache whose
    positions below p0 already hold earlier tokens. The cache rows at the prompt's positions
    hold its roped k and its v, every other row is unchanged, and token t attends causally to
    positions 0..p0 + t (float64 reference from the stored fp16 cache). Cases cover one token,
    a ragged last 16-token block, prompts after a filled prefix, a prompt ending at the cache's
    last position, one kv head per query head and more than 16 query heads per kv head."""
    from kernels.attention import prefill_attention

    g = torch.Generator().manual_seed(p0 + 13 * T + nq)
    hd = 128
    qkv = torch.randn(T, (nq + 2 * nkv) * hd, generator=g).half()
    kc, vc, kt_d, vt_d = _caches(g, nkv, L)
    inv_freq = (1.0 / (1e6 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd)))
    pos = torch.arange(p0, p0 + T, dtype=torch.int64)
    out = prefill_attention(qkv.cuda().view(1, T, -1), pos.cuda(), inv_freq.cuda(), kt_d, vt_d, nq,
                            nkv, hd ** -0.5)
    assert out.shape == (1, T, nq * hd)
    x = qkv.double().numpy()
    fr = inv_freq.numpy()
    k_got = k_from_tiles(kt_d.cpu()).double().numpy()[0]
    v_got = v_from_tiles(vt_d.cpu()).double().numpy()[0]
    new = np.zeros(L, dtype=bool)
    new[p0:p0 + T] = True
    assert np.array_equal(k_got[:, ~new], kc.double().numpy()[0][:, ~new])
    assert np.array_equal(v_got[:, ~new], vc.double().numpy()[0][:, ~new])
    gq = nq // nkv
    got = out.view(T, nq, hd).cpu().double().numpy()
    ref = np.zeros((T, nq, hd))
    for t in range(T):
        p = p0 + t
        k = x[t, nq * hd:(nq + nkv) * hd].reshape(nkv, hd)
        v = x[t, (nq + nkv) * hd:].reshape(nkv, hd)
        kr = _rope64(k, p, fr)
        assert np.abs(k_got[:, p] - kr).max() <= 4e-3 * max(1.0, np.abs(kr).max())
        assert np.array_equal(v_got[:, p], v.astype(np.float16).astype(np.float64))
        qr = _rope64(x[t, : nq * hd].reshape(nq, hd), p, fr)
        for h in range(nq):
            s = k_got[h // gq, : p + 1] @ qr[h] / math.sqrt(hd)
            w = np.exp(s - s.max())
            ref[t, h] = (w / w.sum()) @ v_got[h // gq, : p + 1]
    err = np.abs(got - ref)
    assert err.max() <= 2e-2 and np.linalg.norm(got - ref) / np.linalg.norm(ref) <= 2e-3, (err.max(),)


def test_prefill_positions_out_of_order_and_out_of_range():
    """Each token is masked by its own position, not by its index: a shuffled prompt gives each
    token the row its position gives in order. A position past the cache writes nothing and
    attends to the whole cache; a negative one writes nothing and returns zeros."""
    from kernels.attention import prefill_attention

    nq, nkv, L, T, hd = 12, 2, 96, 40, 128
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(T, (nq + 2 * nkv) * hd, generator=g).half()
    inv = (1.0 / (1e6 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))).cuda()
    perm = torch.randperm(T, generator=g)
    runs = []
    for order in (torch.arange(T), perm):
        _, _, kt, vt = _caches(torch.Generator().manual_seed(9), nkv, L)
        out = prefill_attention(qkv[order].cuda().view(1, T, -1), order.cuda(), inv, kt, vt, nq, nkv,
                                hd ** -0.5)
        runs.append((out[0], kt, vt, order))
    (o0, k0, v0, _), (o1, k1, v1, order) = runs
    assert torch.equal(k0, k1) and torch.equal(v0, v1)
    assert torch.equal(o1, o0[order.cuda()])
    _, _, kt, vt = _caches(torch.Generator().manual_seed(9), nkv, L)
    kt0, vt0 = kt.clone(), vt.clone()
    pos = torch.tensor([L, -1, L + 5], dtype=torch.int64)
    out = prefill_attention(qkv[:3].cuda().view(1, 3, -1), pos.cuda(), inv, kt, vt, nq, nkv, hd ** -0.5)
    assert torch.equal(kt, kt0) and torch.equal(vt, vt0)
    assert torch.isfinite(out).all() and torch.equal(out[0, 1], torch.zeros_like(out[0, 1]))


def _fill_past(kc, vc, last, fill):
    """Copies of the [1, nkv, L, hd] caches with every row past position `last` set to `fill`."""
    k2, v2 = kc.clone(), vc.clone()
    k2[:, :, last + 1:] = fill
    v2[:, :, last + 1:] = fill
    return k_to_tiles(k2).cuda(), vt_to_tiles(v2).cuda()


_FILLS = (0.0, float("nan"), float("inf"), float("-inf"))


@pytest.mark.parametrize("L,pos", [(416, 0), (416, 130), (416, 383), (416, 414), (2144, 2100),
                                   (4096, 1000), (4096, 4000)])
def test_cache_rows_past_pos_can_hold_any_bits(L, pos):
    """The cache rows past pos are not this call's data (an earlier generation's, or never
    written) and may hold any bits. Their softmax weights are 0; the output with NaN or inf in
    them is the output with zeros in them, bit for bit, with one position range (416) and with
    ranges merged by the second launch (2144, 4096). A P.V that multiplied those rows by their
    zero weights would give NaN."""
    nq, nkv, hd = 12, 2, 128
    g = torch.Generator().manual_seed(pos + L)
    qkv = torch.randn((nq + 2 * nkv) * hd, generator=g).half().cuda().view(1, 1, -1)
    kc, vc, _, _ = _caches(g, nkv, L)
    inv = (1.0 / (1e6 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))).cuda()
    p = torch.tensor([pos], device="cuda")
    outs = [decode_attention(qkv, p, inv, *_fill_past(kc, vc, pos, f), nq, nkv, hd ** -0.5) for f in _FILLS]
    assert torch.isfinite(outs[0]).all()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


@pytest.mark.parametrize("p0,T", [(0, 17), (100, 50), (5, 40)])
def test_prefill_cache_rows_past_the_prompt_can_hold_any_bits(p0, T):
    """ldk_prefill_attention: rows past the prompt's last position hold NaN or inf, and every
    token's output is the one with zeros there, bit for bit. In each case the prompt ends inside
    a 32-position chunk, which its last 16-token block reads whole."""
    from kernels.attention import prefill_attention

    nq, nkv, L, hd = 12, 2, 416, 128
    g = torch.Generator().manual_seed(p0 + T)
    qkv = torch.randn(T, (nq + 2 * nkv) * hd, generator=g).half().cuda().view(1, T, -1)
    kc, vc, _, _ = _caches(g, nkv, L)
    inv = (1.0 / (1e6 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))).cuda()
    pos = torch.arange(p0, p0 + T, dtype=torch.int64, device="cuda")
    outs = [prefill_attention(qkv, pos, inv, *_fill_past(kc, vc, p0 + T - 1, f), nq, nkv, hd ** -0.5)
            for f in _FILLS]
    assert torch.isfinite(outs[0]).all()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
