"""Kernel sweep over the benchmark configurations 1-3 on one MI355X (the reference's
kernels/bench/sweep.py case generators, lines 139-207, re-done for this build):

- config 1: fused RMSNorm (with and without residual) at N=1536 and fused SwiGLU at I=8960,
  M in {1, 16, 2048}, seed 1;
- config 2: W4A16 over the six Qwen2.5-1.5B linear shapes at M in {1, 4, 16}, seed 2;
- config 3: W8A16 (OCP e4m3) over the same shapes at M in {1, 4, 8, 16}, seed 3.

- prefill: the W4A16 and W8A16 prefill GEMMs over the Qwen2.5-1.5B projections (qkv fused,
  o, gate_up, down) at M in {512, 2048} (the reference's slow-test rows), as TFLOP/s against the
  2.5 PFLOP/s dense fp16 MFMA peak.

Every case is timed with `harness.GraphTimer` (rotating input sets sized to 4x the 256 MB MALL,
one launch per set in one hipGraph, median of 7 samples) and reported as us, GB/s and % of the
8 TB/s HBM peak with the reference's algorithmic byte formulas. Each row also records the
kernel configuration the library chose. The whole sweep runs `--sweeps` times (3 by default)
and each row reports the median over the sweeps, their min and max, and a flag when the spread
(max - min) / median exceeds 10% (the reference's aggregation, kernels/bench/sweep.py:229-254).

- copy: the practical ceiling, a device-to-device copy (the reference's case, and copies moving as
  many bytes as the two largest decode reads).

    python -m kernels.bench.sweep [--only copy,w4a16,fp8,norm,act,fused,prefill] [--sweeps 3] [--json out.json]
"""

from __future__ import annotations

import argparse
import json
import statistics
import sys

import torch

from kernels.bench import cases
from kernels.bench.harness import GraphTimer, n_copies, tensor_bytes
from kernels.config import GPU_SPECS, PEAK_GBPS

PEAK_FP16_TFLOPS = GPU_SPECS["MI355X"]["peak_fp16_tflops"]

GS = 128


def _time(fn, sets) -> float:
    timer = GraphTimer(fn, sets)
    try:
        return timer.median_ms_per_call()
    finally:
        timer.close()


def _row(kind, shape, M, ms, nbytes, extra=None) -> dict:
    gbps = nbytes / (ms * 1e-3) / 1e9
    r = {"kernel": kind, "shape": shape, "M": M, "us": round(ms * 1e3, 3), "bytes": nbytes,
         "gbps": round(gbps, 1), "pct_peak": round(100 * gbps / PEAK_GBPS, 2)}
    if extra:
        r.update(extra)
    return r


def w4a16_rows(Ms=(1, 2, 4, 8, 16)):
    from kernels.quant import quantize_rtn, weight_bytes
    from kernels.w4a16 import config_for, w4a16_matmul

    rows = []
    for name, N, K in cases.QWEN_LINEARS:
        w, _ = cases.w4a16_case(1, N, K, seed=2)
        qw, s, z = quantize_rtn(w.cuda(), GS)
        for M in Ms:
            x = cases.activations(M, K, cases.gen(2)).cuda()
            per = tensor_bytes((x, qw, s, z)) + 2 * M * N
            sets = [(x.clone(), qw.clone(), s.clone(), z.clone()) for _ in range(n_copies(per))]
            ms = _time(lambda xx, q, sc, zz: w4a16_matmul(xx, q, sc, zz, GS), sets)
            nbytes = weight_bytes(N, K, GS) + 2 * M * K + 2 * M * N  # sweep.py:167-169
            rows.append(_row("w4a16", f"{name} {N}x{K}", M, ms, nbytes,
                             {"config": config_for(M, N, K, GS)}))
            del sets
    return rows


def fp8_rows(Ms=(1, 4, 8, 16)):
    from kernels.fp8 import fp8_bytes, quantize_fp8, w8a16_matmul

    rows = []
    for name, N, K in cases.QWEN_LINEARS:
        w, _ = cases.w4a16_case(1, N, K, seed=3)
        wq, sc = quantize_fp8(w.cuda())
        for M in Ms:
            x = cases.activations(M, K, cases.gen(3)).cuda()
            per = tensor_bytes((x, wq, sc)) + 2 * M * N
            sets = [(x.clone(), wq.clone(), sc.clone()) for _ in range(n_copies(per))]
            ms = _time(lambda xx, q, ss: w8a16_matmul(xx, q, ss), sets)
            nbytes = fp8_bytes(N, K) + 2 * M * K + 2 * M * N  # sweep.py:190-191
            rows.append(_row("w8a16", f"{name} {N}x{K}", M, ms, nbytes))
            del sets
    return rows


def norm_rows(Ms=(1, 16, 2048)):
    from kernels.rmsnorm import rmsnorm, rmsnorm_bytes

    rows = []
    for M in Ms:
        x, r, w = (t.cuda() for t in cases.rmsnorm_case(M, 1536, seed=1))
        for res in (True, False):
            per = tensor_bytes((x, r, w)) * 2
            sets = [(x.clone(), r.clone(), w.clone()) for _ in range(n_copies(per))]
            if res:
                fn = lambda xx, rr, ww: rmsnorm(xx, ww, 1e-6, residual=rr)  # noqa: E731
            else:
                fn = lambda xx, rr, ww: rmsnorm(xx, ww, 1e-6)  # noqa: E731
            ms = _time(fn, sets)
            rows.append(_row("rmsnorm+res" if res else "rmsnorm", "N=1536", M, ms,
                             rmsnorm_bytes(M, 1536, res)))
            del sets
    return rows


def act_rows(Ms=(1, 16, 2048)):
    from kernels.swiglu import swiglu_bytes, swiglu_fused

    rows = []
    for M in Ms:
        gu = cases.swiglu_case(M, 8960, seed=1).cuda()
        sets = [(gu.clone(),) for _ in range(n_copies(tensor_bytes(gu) * 3 // 2))]
        ms = _time(swiglu_fused, sets)
        rows.append(_row("swiglu", "I=8960", M, ms, swiglu_bytes(M, 8960)))
        del sets
    return rows


def fused_rows():
    """The decode layer's fused pairs against their two-launch compositions at M = 1: residual +
    RMSNorm into the qkv (with bias) and gate_up projections, SwiGLU into the down projection.
    Bytes: the projection's plus the activation side's (rmsnorm: x, residual, weight read and the
    new residual written; swiglu: the [2I] row read)."""
    from kernels.fused import rmsnorm_w4a16_matmul, swiglu_w4a16_matmul
    from kernels.quant import quantize_rtn, weight_bytes
    from kernels.rmsnorm import rmsnorm
    from kernels.swiglu import swiglu_fused
    from kernels.w4a16 import w4a16_matmul

    rows = []
    H, I = 1536, 8960
    for name, N, K, bias in (("qkv", 2048, H, True), ("gate_up", 17920, H, False)):
        w, _ = cases.w4a16_case(1, N, K, seed=2)
        qw, s, z = quantize_rtn(w.cuda(), GS)
        b = torch.zeros(N, dtype=torch.float16, device="cuda") if bias else None
        x, r, wn = (t.cuda() for t in cases.rmsnorm_case(1, K, seed=1))
        per = tensor_bytes((x, r, wn, qw, s, z)) + 2 * N + 2 * K
        sets = [(x.clone(), r.clone(), wn.clone(), qw.clone(), s.clone(), z.clone())
                for _ in range(n_copies(per))]
        nbytes = weight_bytes(N, K, GS) + 2 * N + (2 * N if bias else 0) + 4 * K * 2 + 2 * K

        def fused(xx, rr, ww, q, sc, zz):
            return rmsnorm_w4a16_matmul(xx, ww, 1e-6, rr, q, sc, zz, GS, b)

        def split(xx, rr, ww, q, sc, zz):
            h, res = rmsnorm(xx, ww, 1e-6, residual=rr)
            return w4a16_matmul(h, q, sc, zz, GS, b), res

        for kind, fn in (("rms+w4a16", fused), ("rms,w4a16", split)):
            rows.append(_row(kind, f"{name} {N}x{K}", 1, _time(fn, sets), nbytes))
        del sets
    w, _ = cases.w4a16_case(1, H, I, seed=2)
    qw, s, z = quantize_rtn(w.cuda(), GS)
    gu = cases.swiglu_case(1, I, seed=1).cuda()
    per = tensor_bytes((gu, qw, s, z)) + 2 * H
    sets = [(gu.clone(), qw.clone(), s.clone(), z.clone()) for _ in range(n_copies(per))]
    nbytes = weight_bytes(H, I, GS) + 2 * H + 4 * I
    rows.append(_row("swiglu+w4a16", f"down {H}x{I}", 1,
                     _time(lambda g, q, sc, zz: swiglu_w4a16_matmul(g, q, sc, zz, GS), sets), nbytes))
    rows.append(_row("swiglu,w4a16", f"down {H}x{I}", 1,
                     _time(lambda g, q, sc, zz: w4a16_matmul(swiglu_fused(g), q, sc, zz, GS), sets),
                     nbytes))
    del sets
    return rows


def copy_rows():
    """The practical ceiling: a device-to-device copy (dst.copy_(src)), the reference's copy case
    (kernels/bench/sweep.py:61-70: 64M fp16 elements, 128 MiB read and 128 MiB written), and
    copies that move as many bytes as the decode kernels' two largest reads (config 0's
    14,661,632 B and down's 7,332,352 B, half read and half written), on rotating sets like every
    other row. Bytes are read plus written (2 * 2 * elems)."""
    rows = []
    for label, n in (("ref 64M fp16", 64 * 2**20), ("= gate_up M=1 bytes", 14_661_632 // 4),
                     ("= down M=1 bytes", 7_332_352 // 4)):
        src = torch.randn(n, dtype=torch.float16, device="cuda")
        sets = [(src.clone(), torch.empty_like(src)) for _ in range(n_copies(4 * n))]
        del src
        ms = _time(lambda a, b: b.copy_(a), sets)
        rows.append(_row("copy", f"{label} ({n})", 1, ms, 2 * n * 2))
        del sets
    return rows


PREFILL_SHAPES = [("qkv", 2048, 1536), ("o", 1536, 1536), ("gate_up", 17920, 1536), ("down", 1536, 8960)]


def _flops_extra(M, N, K, ms) -> dict:
    tflops = 2 * M * N * K / (ms * 1e-3) / 1e12
    return {"flops": 2 * M * N * K, "tflops": round(tflops, 1),
            "pct_mfma": round(100 * tflops / PEAK_FP16_TFLOPS, 2)}


def prefill_rows(Ms=(512, 2048)):
    """The prefill GEMMs (the library's choice for these rows) at the reference's slow-test row
    counts; bytes are the weights, x and y once each."""
    from kernels.fp8 import fp8_bytes, quantize_fp8, w8a16_matmul
    from kernels.quant import quantize_rtn, weight_bytes
    from kernels.w4a16 import kernel_name, w4a16_matmul

    rows = []
    for name, N, K in PREFILL_SHAPES:
        w, _ = cases.w4a16_case(1, N, K, seed=2)
        qw, s, z = quantize_rtn(w.cuda(), GS)
        wq, sc = quantize_fp8(w.cuda())
        for M in Ms:
            x = cases.activations(M, K, cases.gen(2)).cuda()
            sets = [(x.clone(), qw.clone(), s.clone(), z.clone())
                    for _ in range(n_copies(tensor_bytes((x, qw, s, z)) + 2 * M * N))]
            ms = _time(lambda xx, q, ss, zz: w4a16_matmul(xx, q, ss, zz, GS), sets)
            extra = {"config": kernel_name(M, N, K, GS), **_flops_extra(M, N, K, ms)}
            rows.append(_row("w4a16 gemm", f"{name} {N}x{K}", M, ms,
                             weight_bytes(N, K, GS) + 2 * M * K + 2 * M * N, extra))
            sets = [(x.clone(), wq.clone(), sc.clone())
                    for _ in range(n_copies(tensor_bytes((x, wq, sc)) + 2 * M * N))]
            ms = _time(lambda xx, q, ss: w8a16_matmul(xx, q, ss), sets)
            rows.append(_row("w8a16 gemm", f"{name} {N}x{K}", M, ms,
                             fp8_bytes(N, K) + 2 * M * K + 2 * M * N, _flops_extra(M, N, K, ms)))
            del sets
    return rows


SECTIONS = {"copy": copy_rows, "w4a16": w4a16_rows, "fp8": fp8_rows, "norm": norm_rows, "act": act_rows,
            "fused": fused_rows, "prefill": prefill_rows}


def aggregate(sweeps: list[list[dict]]) -> list[dict]:
    """Median over sweeps per row (every sweep lists the same cases in the same order), with the
    min, max and a >10% spread flag (kernels/bench/sweep.py:229-254 of the reference)."""
    out = []
    for rs in zip(*sweeps):
        us = [r["us"] for r in rs]
        med = statistics.median(us)
        row = _row(rs[0]["kernel"], rs[0]["shape"], rs[0]["M"], med * 1e-3, rs[0]["bytes"])
        for k in ("config", "flops"):
            if k in rs[0]:
                row[k] = rs[0][k]
        if "flops" in row:
            row.update(_flops_extra(1, row["flops"] // 2, 1, med * 1e-3))
        spread = 100 * (max(us) - min(us)) / med
        row.update({"sweeps": len(us), "us_min": min(us), "us_max": max(us),
                    "spread_pct": round(spread, 2), "flag_spread": spread > 10})
        out.append(row)
    return out


def _line(r) -> str:
    t = f"  {r['tflops']:7.1f} TFLOP/s {r['pct_mfma']:5.2f}%" if "tflops" in r else ""
    agg = f"  [{r['us_min']:.3f}-{r['us_max']:.3f}{' SPREAD' if r['flag_spread'] else ''}]" if "sweeps" in r else ""
    return (f"{r['kernel']:12s} {r['shape']:22s} M={r['M']:<5d} {r['us']:9.3f} us "
            f"{r['gbps']:8.1f} GB/s {r['pct_peak']:6.2f}%{t}{agg}  {r.get('config', '')}")


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--only", default="copy,w4a16,fp8,norm,act")
    ap.add_argument("--sweeps", type=int, default=3)
    ap.add_argument("--json", default=None)
    args = ap.parse_args(argv)
    torch.cuda.init()
    sweeps = []
    for i in range(args.sweeps):
        rows = []
        for sec in args.only.split(","):
            for r in SECTIONS[sec]():
                print(f"[sweep {i + 1}/{args.sweeps}] " + _line(r), flush=True)
                rows.append(r)
        sweeps.append(rows)
    agg = aggregate(sweeps)
    print(f"median of {args.sweeps} sweeps:")
    for r in agg:
        print(_line(r), flush=True)
    if args.json:
        with open(args.json, "w") as f:
            json.dump({"peak_gbps": PEAK_GBPS, "peak_fp16_tflops": PEAK_FP16_TFLOPS,
                       "sweeps": args.sweeps, "rows": agg, "per_sweep": sweeps}, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
