"""Counter workload: launches each hot-path kernel on the benchmark configurations so that one
rocprofv3 run per counter set covers all of them, plus a 64 MiB elementwise pass (torch.neg on
fp16) that calibrates the byte counters: it reads and writes exactly 65536 KiB per dispatch.

Every case rotates over input sets sized to 4x the 256 MB MALL (as the sweep does), so each
launch reads its weights from HBM. Cases run one after another, `--reps` launches each.

    rocprofv3 --kernel-trace --stats -d OUT -o prof -- python3 -m kernels.bench.profile_cases
    rocprofv3 --pmc FETCH_SIZE -d OUT -o prof -- python3 -m kernels.bench.profile_cases
    rocprofv3 --pmc WRITE_SIZE -d OUT -o prof -- python3 -m kernels.bench.profile_cases
    rocprofv3 --pmc VALUBusy MfmaUtil -d OUT -o prof -- python3 -m kernels.bench.profile_cases
    python3 -m kernels.bench.counters OUT        # one table per kernel and grid

`--cases` picks a subset by name (comma-separated). `--graph` times each case instead, in hipGraph
replays over the same rotating sets (the sweep's method), and prints microseconds per launch.
"""

from __future__ import annotations

import argparse

import torch

from kernels.bench import cases
from kernels.bench.harness import n_copies, tensor_bytes

GS = 128


GRAPH = False  # --graph: time each case in hipGraph replays instead of launching it eagerly


def _rotate(fn, sets, reps):
    if GRAPH:
        from kernels.bench.harness import GraphTimer

        timer = GraphTimer(fn, sets)
        try:
            print(f"  graph-timed: {timer.median_ms_per_call() * 1e3:.3f} us per launch", flush=True)
        finally:
            timer.close()
        return
    for i in range(reps):
        fn(*sets[i % len(sets)])


def case_w4a16(M, N, K, reps, config=None):
    from kernels.quant import quantize_rtn
    from kernels.w4a16 import w4a16_matmul

    w, _ = cases.w4a16_case(1, N, K, seed=2)
    qw, s, z = quantize_rtn(w.cuda(), GS)
    x = cases.activations(M, K, cases.gen(2)).cuda()
    sets = [(x.clone(), qw.clone(), s.clone(), z.clone())
            for _ in range(n_copies(tensor_bytes((x, qw, s, z))))]
    _rotate(lambda xx, q, sc, zz: w4a16_matmul(xx, q, sc, zz, GS, config=config), sets, reps)


def case_fp8(M, N, K, reps):
    from kernels.fp8 import quantize_fp8, w8a16_matmul

    w, _ = cases.w4a16_case(1, N, K, seed=3)
    wq, sc = quantize_fp8(w.cuda())
    x = cases.activations(M, K, cases.gen(3)).cuda()
    sets = [(x.clone(), wq.clone(), sc.clone()) for _ in range(n_copies(tensor_bytes((x, wq, sc))))]
    _rotate(lambda xx, q, ss: w8a16_matmul(xx, q, ss), sets, reps)


def case_rms_w4a16(N, K, reps, bias):
    from kernels.fused import rmsnorm_w4a16_matmul
    from kernels.quant import quantize_rtn

    w, _ = cases.w4a16_case(1, N, K, seed=2)
    qw, s, z = quantize_rtn(w.cuda(), GS)
    b = torch.zeros(N, dtype=torch.float16, device="cuda") if bias else None
    x, r, wn = (t.cuda() for t in cases.rmsnorm_case(1, K, seed=1))
    sets = [(x.clone(), r.clone(), qw.clone(), s.clone(), z.clone())
            for _ in range(n_copies(tensor_bytes((x, r, qw, s, z))))]
    _rotate(lambda xx, rr, q, sc, zz: rmsnorm_w4a16_matmul(xx, wn, 1e-6, rr, q, sc, zz, GS, b),
            sets, reps)


def case_swiglu_w4a16(N, I, reps):
    from kernels.fused import swiglu_w4a16_matmul
    from kernels.quant import quantize_rtn

    w, _ = cases.w4a16_case(1, N, I, seed=2)
    qw, s, z = quantize_rtn(w.cuda(), GS)
    gu = cases.swiglu_case(1, I, seed=1).cuda()
    sets = [(gu.clone(), qw.clone(), s.clone(), z.clone())
            for _ in range(n_copies(tensor_bytes((gu, qw, s, z))))]
    _rotate(lambda g, q, sc, zz: swiglu_w4a16_matmul(g, q, sc, zz, GS), sets, reps)


def case_linear_rms_pair(reps):
    """o projection (residual add and per-tile sums of squares in its epilogue) into gate_up
    (RMSNorm formed in its staging from those sums), at the Qwen2.5-1.5B shapes."""
    from kernels.fused import linear_rmsnorm_w4a16_matmul
    from kernels.quant import quantize_rtn

    H, I2 = 1536, 17920
    w1, _ = cases.w4a16_case(1, H, H, seed=2)
    w2, _ = cases.w4a16_case(1, I2, H, seed=3)
    q1, s1, z1 = quantize_rtn(w1.cuda(), GS)
    q2, s2, z2 = quantize_rtn(w2.cuda(), GS)
    x, r, wn = (t.cuda() for t in cases.rmsnorm_case(1, H, seed=1))
    sets = [(q1.clone(), s1.clone(), z1.clone(), q2.clone(), s2.clone(), z2.clone())
            for _ in range(n_copies(tensor_bytes((q1, s1, z1, q2, s2, z2))))]
    _rotate(lambda a, b, c, d, e, f: linear_rmsnorm_w4a16_matmul(
        x, a, b, c, None, r, wn, 1e-6, d, e, f, None, GS), sets, reps)


def case_rms_fp8(N, K, reps):
    from kernels.fp8 import quantize_fp8
    from kernels.fused import rmsnorm_w8a16_matmul

    w, _ = cases.w4a16_case(1, N, K, seed=3)
    wq, sc = quantize_fp8(w.cuda())
    x, r, wn = (t.cuda() for t in cases.rmsnorm_case(1, K, seed=1))
    sets = [(wq.clone(), sc.clone()) for _ in range(n_copies(tensor_bytes((wq, sc))))]
    _rotate(lambda q, ss: rmsnorm_w8a16_matmul(x, wn, 1e-6, r, q, ss), sets, reps)


def case_swiglu_fp8(N, I, reps):
    from kernels.fp8 import quantize_fp8
    from kernels.fused import swiglu_w8a16_matmul

    w, _ = cases.w4a16_case(1, N, I, seed=3)
    wq, sc = quantize_fp8(w.cuda())
    gu = cases.swiglu_case(1, I, seed=1).cuda()
    sets = [(wq.clone(), sc.clone()) for _ in range(n_copies(tensor_bytes((wq, sc))))]
    _rotate(lambda q, ss: swiglu_w8a16_matmul(gu, q, ss), sets, reps)


def case_attention(reps, L=416, pos=300):
    from kernels.attention import decode_attention, k_cache_shape, vt_cache_shape

    g = cases.gen(5)
    nq, nkv, hd = 12, 2, 128
    qkv = torch.randn((nq + 2 * nkv) * hd, generator=g).half().cuda()
    kc = torch.randn((1,) + k_cache_shape(nkv, L), generator=g).half().cuda()
    vt = torch.randn((1,) + vt_cache_shape(nkv, L), generator=g).half().cuda()
    inv = (1.0 / (1e6 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))).cuda()
    p = torch.tensor([pos], device="cuda")
    sets = [(kc.clone(), vt.clone()) for _ in range(n_copies(tensor_bytes((kc, vt))))]
    _rotate(lambda k, v: decode_attention(qkv, p, inv, k, v, nq, nkv, hd ** -0.5), sets, reps)


def case_prefill_attention(reps, T=128, L=416):
    """The prompt's attention block (kernels.attention.prefill_attention): T tokens at positions
    0..T-1 of a cache of L, Qwen2.5-1.5B heads (12 / 2 of 128)."""
    from kernels.attention import k_cache_shape, prefill_attention, vt_cache_shape

    g = cases.gen(6)
    nq, nkv, hd = 12, 2, 128
    qkv = torch.randn(1, T, (nq + 2 * nkv) * hd, generator=g).half().cuda()
    kc = torch.randn((1,) + k_cache_shape(nkv, L), generator=g).half().cuda()
    vt = torch.randn((1,) + vt_cache_shape(nkv, L), generator=g).half().cuda()
    inv = (1.0 / (1e6 ** (torch.arange(0, hd, 2, dtype=torch.float32) / hd))).cuda()
    p = torch.arange(T, device="cuda")
    sets = [(kc.clone(), vt.clone()) for _ in range(n_copies(tensor_bytes((kc, vt))))]
    _rotate(lambda k, v: prefill_attention(qkv, p, inv, k, v, nq, nkv, hd ** -0.5), sets, reps)


def case_prefill_forward(reps, backend="ours", T=128):
    """The config-4 runner's prompt forward (random-init Qwen2.5-1.5B architecture, seed 4, a
    T-token prompt at positions 0..T-1), eager, reps times: every prefill launch of a layer."""
    from kernels.e2e.model import QwenRunner, make_backend, random_qwen2

    hf = random_qwen2(seed=4)
    ids = torch.randint(0, hf.config.vocab_size, (1, T), device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(4))
    runner = QwenRunner(hf, make_backend(backend), max_len=416)
    pos = torch.arange(T, device="cuda")
    for _ in range(reps):
        runner.forward(ids, pos)


def case_rmsnorm(M, N, reps):
    from kernels.rmsnorm import rmsnorm

    x, r, w = (t.cuda() for t in cases.rmsnorm_case(M, N, seed=1))
    sets = [(x.clone(), r.clone()) for _ in range(n_copies(tensor_bytes((x, r)) * 2))]
    _rotate(lambda xx, rr: rmsnorm(xx, w, 1e-6, residual=rr), sets, reps)


def case_swiglu(M, I, reps):
    from kernels.swiglu import swiglu_fused

    gu = cases.swiglu_case(M, I, seed=1).cuda()
    sets = [(gu.clone(),) for _ in range(n_copies(tensor_bytes(gu) * 3 // 2))]
    _rotate(swiglu_fused, sets, reps)


def case_copy(reps):
    """torch.neg over 64 MiB of fp16: reads and writes exactly 65536 KiB per dispatch, under a
    kernel name nothing else in the workload uses (the weight clones run rocclr's copy kernel)."""
    a = torch.randn(32 * 2**20, dtype=torch.float16, device="cuda")
    b = torch.empty_like(a)
    for _ in range(reps):
        torch.neg(a, out=b)


CASES = {
    "calib_neg64MiB": lambda r: case_copy(r),
    "w4a16_gate_up_m1": lambda r: case_w4a16(1, 17920, 1536, r),
    "prefill_forward_ours": lambda r: case_prefill_forward(r, "ours"),
    "prefill_forward_ours_fp8": lambda r: case_prefill_forward(r, "ours_fp8"),
    # the M = 1 kernel and the read floors at K = 1536 and wider N (2x, 4x gate_up, and the
    # 151936-row vocabulary of the quantized lm_head): where launch and ramp stop dominating
    **{f"w4a16_m1_n{n}": (lambda r, n=n: case_w4a16(1, n, 1536, r)) for n in (35840, 71680, 151936)},
    "w4a16_down_m1": lambda r: case_w4a16(1, 1536, 8960, r),
    "w4a16_gate_up_m2": lambda r: case_w4a16(2, 17920, 1536, r),
    "w4a16_gate_up_m4": lambda r: case_w4a16(4, 17920, 1536, r),
    "w4a16_gate_up_m16": lambda r: case_w4a16(16, 17920, 1536, r),
    "w4a16_down_m16": lambda r: case_w4a16(16, 1536, 8960, r),
    "fp8_gate_up_m1": lambda r: case_fp8(1, 17920, 1536, r),
    "fp8_gate_up_m16": lambda r: case_fp8(16, 17920, 1536, r),
    # decode rows of the other shapes: W4A16 down at two rows (MFMA), FP8 at 4 and 16 rows
    "w4a16_down_m2": lambda r: case_w4a16(2, 1536, 8960, r),
    "fp8_gate_up_m4": lambda r: case_fp8(4, 17920, 1536, r),
    "fp8_down_m4": lambda r: case_fp8(4, 1536, 8960, r),
    "fp8_down_m16": lambda r: case_fp8(16, 1536, 8960, r),
    "fp8_o_m16": lambda r: case_fp8(16, 1536, 1536, r),
    "fp8_k_m16": lambda r: case_fp8(16, 256, 1536, r),
    "rms_qkv_m1": lambda r: case_rms_w4a16(2048, 1536, r, True),
    "rms_gate_up_m1": lambda r: case_rms_w4a16(17920, 1536, r, False),
    "swiglu_down_m1": lambda r: case_swiglu_w4a16(1536, 8960, r),
    "o_rms_gate_up_pair_m1": lambda r: case_linear_rms_pair(r),
    "fp8_rms_gate_up_m1": lambda r: case_rms_fp8(17920, 1536, r),
    "fp8_swiglu_down_m1": lambda r: case_swiglu_fp8(1536, 8960, r),
    "attention_l416": lambda r: case_attention(r),
    "attention_l4096": lambda r: case_attention(r, L=4096, pos=4000),
    "prefill_attention_t128": lambda r: case_prefill_attention(r),
    # prefill rows of down on the 32-row MFMA blocks with K split over workgroups
    "w4a16_down_m65": lambda r: case_w4a16(65, 1536, 8960, r),
    "w4a16_down_m128": lambda r: case_w4a16(128, 1536, 8960, r),
    "rmsnorm_res_m2048": lambda r: case_rmsnorm(2048, 1536, r),
    "swiglu_m2048": lambda r: case_swiglu(2048, 8960, r),
    # decode rows 4 and 8 on the VALU kernel (forced) against the library's MFMA kernel
    "w4a16_gate_up_m4_valu": lambda r: case_w4a16(4, 17920, 1536, r, {"GEMV": True}),
    "w4a16_gate_up_m8": lambda r: case_w4a16(8, 17920, 1536, r),
    "w4a16_gate_up_m8_valu": lambda r: case_w4a16(8, 17920, 1536, r, {"GEMV": True}),
    "w4a16_down_m4": lambda r: case_w4a16(4, 1536, 8960, r),
    "w4a16_down_m4_valu": lambda r: case_w4a16(4, 1536, 8960, r, {"GEMV": True}),
    # decode rows 4-16: the library's x-staged MFMA kernel against the wide-tile MFMA kernel (forced)
    "w4a16_gate_up_m4_wide": lambda r: case_w4a16(4, 17920, 1536, r, {"MFMA": True, "block_n": 128}),
    "w4a16_gate_up_m16_wide": lambda r: case_w4a16(16, 17920, 1536, r, {"MFMA": True, "block_n": 128}),
    "w4a16_o_m16": lambda r: case_w4a16(16, 1536, 1536, r),
    "w4a16_o_m16_wide": lambda r: case_w4a16(16, 1536, 1536, r, {"MFMA": True, "block_n": 32}),
    "w4a16_k_m16": lambda r: case_w4a16(16, 256, 1536, r),
    "w4a16_k_m16_wide": lambda r: case_w4a16(16, 256, 1536, r, {"MFMA": True, "block_n": 32}),
    # prefill GEMMs (the library's choice at these rows)
    "w4a16_qkv_m2048": lambda r: case_w4a16(2048, 2048, 1536, r),
    "w4a16_o_m2048": lambda r: case_w4a16(2048, 1536, 1536, r),
    "w4a16_gate_up_m2048": lambda r: case_w4a16(2048, 17920, 1536, r),
    "w4a16_down_m2048": lambda r: case_w4a16(2048, 1536, 8960, r),
    "w4a16_gate_up_m512": lambda r: case_w4a16(512, 17920, 1536, r),
    "fp8_qkv_m2048": lambda r: case_fp8(2048, 2048, 1536, r),
    "fp8_o_m2048": lambda r: case_fp8(2048, 1536, 1536, r),
    "fp8_gate_up_m2048": lambda r: case_fp8(2048, 17920, 1536, r),
    "fp8_down_m2048": lambda r: case_fp8(2048, 1536, 8960, r),
}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reps", type=int, default=40)
    ap.add_argument("--cases", default=",".join(CASES))
    ap.add_argument("--graph", action="store_true",
                    help="time each case in hipGraph replays (kernels.bench.harness.GraphTimer)")
    args = ap.parse_args(argv)
    global GRAPH
    GRAPH = args.graph
    torch.cuda.init()
    for name in args.cases.split(","):
        print(f"case {name}:", flush=True)
        CASES[name](args.reps)
        torch.cuda.synchronize()
        if not GRAPH:
            print(f"  {args.reps} launches", flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
