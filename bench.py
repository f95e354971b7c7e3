"""Headline benchmark: W4A16 GEMV at M=1 on the Qwen2.5-1.5B gate_up shape (config 0) on one
MI355X, as HBM GB/s and fraction of the 8 TB/s roofline, with the oracle's CPU path timed beside
it on the host cores.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-e2e]

A step is one W4A16 launch over one rotating input set (x, qweight, scales, zeros, output); the
sets are sized to 4x the 256 MB MALL so every step reads its weights from HBM. Steps run as
hipGraph replays of one launch per set; HIP events on the replay stream bracket the timed steps.
The config-4 decode (fp16 vs swapped tok/s) and the CPU baseline are reported beside it.
Prints one JSON line.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "llm-decode-kernels_amd"))

METRIC = "W4A16 M=1 HBM GB/s & % of peak; Qwen2.5-1.5B-arch batch-1 decode tok/s"
M, N, K, GS, SEED = 1, 17920, 1536, 128, 0


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def cpu_baseline(w16, x, seconds: float = 15.0) -> dict:
    """The oracle's restatement of the reference CPU path (kernels/reference.py:39-45: unpack and
    dequantize every call, then the fp32 matmul), single-threaded, on a bounded sample of calls:
    3 warm-up calls, then timed calls until ~`seconds` of CPU work (at most 7, median). Beside it,
    the dequantize-once variant (the reference's W4RefBackend, e2e/model.py:62-67): the fp32
    matmul alone over weights dequantized beforehand."""
    from threadpoolctl import threadpool_limits

    from oracle import quant as oq
    from oracle.reference import w4a16_ref

    qw, s, z = oq.quantize_rtn(w16.numpy(), GS)
    xn = x.numpy()
    with threadpool_limits(limits=1):
        t0 = time.perf_counter()
        w4a16_ref(xn, qw, s, z, GS)
        one = time.perf_counter() - t0
        warm = 0 if one * 3 > seconds / 2 else 2
        for _ in range(warm):
            w4a16_ref(xn, qw, s, z, GS)
        n = int(max(1, min(7, (seconds - one * (1 + warm)) // max(one, 1e-6))))
        times = []
        for _ in range(n):
            t0 = time.perf_counter()
            w4a16_ref(xn, qw, s, z, GS)
            times.append(time.perf_counter() - t0)
        # dequantize once (as the reference's W4RefBackend, model.py:62-67), then fp32 matmuls
        from oracle.reference import dequantize_ref

        w32 = dequantize_ref(qw, s, z, GS).astype("float32")
        x32 = xn.astype("float32")
        once = []
        for _ in range(10):
            t0 = time.perf_counter()
            _ = x32 @ w32.T
            once.append(time.perf_counter() - t0)
    from kernels.quant import weight_bytes

    sec = statistics.median(times)
    nbytes = weight_bytes(N, K, GS) + 2 * M * K + 2 * M * N
    sec_once = statistics.median(once[3:])
    return {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{len(times)} timed calls (+{1 + warm} warm-up) of oracle w4a16_ref on "
                      f"config 0 (dequantize each call + fp32 matmul), median "
                      f"{sec * 1e3:.1f} ms/call, 1 thread of {os.cpu_count()} "
                      f"({_cpu_model()})",
            "dequant_once": {"value": round(nbytes / sec_once / 1e9, 3), "unit": "GB/s",
                             "sample": f"weights dequantized once to fp32 outside the timing, "
                                       f"then 7 timed fp32 matmuls (+3 warm-up), median "
                                       f"{sec_once * 1e3:.2f} ms/call, 1 thread (same "
                                       f"algorithmic bytes as the int4 path)"}}


def e2e_leg(steps: int) -> dict:
    """Config 4, the metric's second half: batch-1 greedy decode of the random-init
    Qwen2.5-1.5B architecture (seed 4), 128-token prompt then `steps` decode steps, each step one
    hipGraph replay; fp16 library GEMMs against the swapped W4A16/RMSNorm/SwiGLU kernels (`ours`,
    fp16 tied lm_head as in the reference; `ours_lm`, lm_head quantized too). Reported beside the
    headline, not as `value`."""
    import gc

    import torch

    from kernels.e2e.run import run

    res = run({"backends": ["fp16", "ours", "ours_lm"], "decode_steps": steps, "prompt_len": 128})
    gc.collect()
    torch.cuda.empty_cache()
    b = res["backends"]
    return {"metric": "Qwen2.5-1.5B-arch batch-1 decode tok/s", "unit": "tok/s",
            "workload": "random-init Qwen2.5-1.5B architecture (seed 4), prompt 128, "
                        f"{steps} greedy steps, hipGraph per step, median of 3",
            "tok_s": {k: round(v["decode"]["tok_s"], 1) for k, v in b.items()},
            "ms_per_token": {k: round(v["decode"]["ms_per_token"], 3) for k, v in b.items()},
            "layers_only_ms": {k: round(v["layers_only_ms"], 3) for k, v in b.items()},
            "speedup_vs_fp16": {k: round(v["speedup_vs_fp16"], 3) for k, v in b.items()},
            "linear_bytes_per_token": {k: v["weights"]["linear_layers"] for k, v in b.items()}}


def measured_traffic(kernel_config: str):
    """HBM bytes per launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary of this
    command (profiles/w4a16_m1_gate_up_traffic.md), or None when that summary was taken with a
    different kernel configuration than the one the library chooses now."""
    path = REPO / "profiles" / "w4a16_m1_gate_up_traffic.md"
    try:
        text = path.read_text()
    except OSError:
        return None
    fields = {}
    for line in text.splitlines():
        if ":" in line and line.split(":", 1)[0] in ("traffic_bytes_per_launch", "kernel_config"):
            k, v = line.split(":", 1)
            fields[k] = v.strip()
    if fields.get("kernel_config") != kernel_config or "traffic_bytes_per_launch" not in fields:
        return None
    return int(fields["traffic_bytes_per_launch"])


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20000)
    ap.add_argument("--warmup", type=int, default=500)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-e2e", action="store_true",
                    help="skip the config-4 decode leg (fp16 vs swapped tok/s)")
    ap.add_argument("--e2e-steps", type=int, default=256)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the W4A16 path would shard by output columns with no exchange; see DESIGN.md)",
              file=sys.stderr)
        return 2

    import torch

    from kernels.bench import cases
    from kernels.bench.harness import GraphTimer, n_copies
    from kernels.config import PEAK_GBPS
    from kernels.quant import quantize_rtn, weight_bytes
    from kernels.w4a16 import config_for, w4a16_matmul

    torch.cuda.init()
    w16, x = cases.w4a16_case(M, N, K, SEED)
    qw, s, z = quantize_rtn(w16.cuda(), GS)
    xg = x.cuda()
    set_bytes = sum(t.numel() * t.element_size() for t in (qw, s, z, xg)) + 2 * M * N
    ncopy = n_copies(set_bytes)
    sets = [(xg.clone(), qw.clone(), s.clone(), z.clone()) for _ in range(ncopy)]
    del qw, s, z

    def step(xx, q, sc, zz):
        return w4a16_matmul(xx, q, sc, zz, GS)

    timer = GraphTimer(step, sets)
    per_replay = timer.calls_per_replay
    warm_replays = max(1, math.ceil(args.warmup / per_replay))
    timer.time_replays(warm_replays)
    replays = max(1, math.ceil(args.steps / per_replay))
    torch.cuda.synchronize()
    total_ms = timer.time_replays(replays)
    torch.cuda.synchronize()
    steps = replays * per_replay
    ms_per_step = total_ms / steps

    nbytes = weight_bytes(N, K, GS) + 2 * M * K + 2 * M * N  # sweep.py:167-169
    gbps = nbytes / (ms_per_step * 1e-3) / 1e9
    kcfg = config_for(M, N, K, GS)
    out = {
        "metric": METRIC,
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm_replays * per_replay,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seed 0: W ~ N(0,0.02) fp16 RTN-quantized on the GPU, x ~ N(0,1))",
        "config": {"workload": "W4A16 GEMV, M=1, N=17920, K=1536 (Qwen2.5-1.5B gate_up), "
                               "group 128 (config 0)",
                   "M": M, "N": N, "K": K, "group_size": GS, "rotating_sets": ncopy,
                   "kernel_config": kcfg},
        "pct_of_peak": round(100 * gbps / PEAK_GBPS, 2),
        "us_per_call": round(ms_per_step * 1e3, 3),
        "roofline": {"bound": "hbm", "achieved": round(gbps, 2), "peak": PEAK_GBPS,
                     "unit": "GB/s", "frac": round(gbps / PEAK_GBPS, 4),
                     "traffic": measured_traffic(kcfg), "bytes_per_launch": nbytes,
                     "kernel": "w4a16_m1_kernel<8, 6, 4, 0, 1>",
                     "timing": "HIP events on the graph-replay stream over all timed launches"},
    }
    timer.close()
    del sets
    if not args.no_e2e:
        out["e2e"] = e2e_leg(args.e2e_steps)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(w16, x)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
