"""Headline benchmark: W4A16 GEMV at M=1 on the Qwen2.5-1.5B gate_up shape (config 0) on one
MI355X, as HBM GB/s and fraction of the 8 TB/s roofline, with the reference's CPU path (restated
in torch, oracle/torch_cpu.py) timed beside it on the host cores.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-e2e]

A step is one W4A16 launch over one rotating input set (x, qweight, scales, zeros, output); the
sets are sized to 4x the 256 MB MALL so every step reads its weights from HBM. Steps run as
hipGraph replays of one launch per set, HIP events on the replay stream. The --warmup W untimed
launches run as whole replays (W rounded up; the count run is reported as timed.warmup_launches,
while "warmup" echoes W as requested). The timed region holds
7 samples, each of at least max(K, 50 ms worth of) launches in whole replays; ms_per_step is the
median sample's time per launch. The config-4 decode (fp16 vs swapped tok/s) and the CPU
baseline are reported beside it. Prints one JSON line.
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
SAMPLES, MIN_SAMPLE_MS = 7, 50.0


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def usable_cpus() -> int:
    """CPUs this process may run on: its affinity set, capped by a cgroup CPU quota if any."""
    n = len(os.sched_getaffinity(0))
    try:
        quota, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if quota != "max":
            n = min(n, max(1, int(int(quota) // int(period))))
    except (OSError, ValueError):
        pass
    return n


def _time_cpu(fn, budget_s: float = 4.0) -> tuple[float, int]:
    """Median seconds per call: 3 warm-ups then 7 timed calls, fewer when one call is long
    (1 warm-up and 3 timed calls above budget_s / 4 per call)."""
    t0 = time.perf_counter()
    fn()
    one = time.perf_counter() - t0
    warm, timed = (3, 7) if one * 10 <= budget_s else (1, 3)
    for _ in range(warm - 1):
        fn()
    times = []
    for _ in range(timed):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), timed


def cpu_baseline(w16, x) -> dict:
    """The reference's CPU path (kernels/reference.py:9-45, fp8.py:33-35) as torch ops on the host
    (oracle/torch_cpu.py, pinned against the numpy oracle), on every usable core. Headline: config
    0 through the full reference path (unpack + dequantize every call, then the fp32 matmul), in
    the metric's unit. Rows beside it: the dequantize-once variant (the reference's W4RefBackend,
    e2e/model.py:62-67), RMSNorm (+ residual) and SwiGLU (config 1) and the FP8 path (config 3's
    gate_up, dequantize every call) at M in {1, 16, 2048}."""
    import torch

    from kernels.bench import cases
    from oracle import fp8 as of
    from oracle import quant as oq
    from oracle import torch_cpu as tc

    threads = usable_cpus()
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    t_start = time.perf_counter()
    try:
        qw, s, z = (torch.from_numpy(a) for a in oq.quantize_rtn(w16.numpy(), GS))
        nbytes = 14_622_720 + 2 * M * K + 2 * M * N  # weight_bytes(N, K) + x + y (sweep.py:167-169)
        sec, n = _time_cpu(lambda: tc.w4a16_ref(x, qw, s, z, GS))
        w32 = tc.dequantize_ref(qw, s, z, GS).float()
        sec_once, n_once = _time_cpu(lambda: torch.matmul(x.float(), w32.t()))
        rows = {"w4a16_dequant_once": {"M": 1, "ms": round(sec_once * 1e3, 3),
                                       "GB/s": round(nbytes / sec_once / 1e9, 3)}}
        wq8, sc8 = of.quantize_fp8(w16.numpy())
        wq8 = torch.from_numpy(wq8).view(torch.float8_e4m3fn)
        sc8 = torch.from_numpy(sc8)
        for m in (1, 16, 2048):
            xr, r, wr = cases.rmsnorm_case(m, 1536, seed=1)
            t_rms, _ = _time_cpu(lambda: tc.rmsnorm_ref(xr, wr, 1e-6, residual=r))
            b = 4 * m * 1536 * 2 + 2 * 1536  # rmsnorm.py:71-74 with the residual
            rows[f"rmsnorm_res_M{m}"] = {"ms": round(t_rms * 1e3, 4), "GB/s": round(b / t_rms / 1e9, 3)}
            gu = cases.swiglu_case(m, 8960, seed=1)
            g, u = gu[:, :8960], gu[:, 8960:]
            t_sw, _ = _time_cpu(lambda: tc.swiglu_ref(g, u))
            b = 3 * m * 8960 * 2  # swiglu.py:64-65
            rows[f"swiglu_M{m}"] = {"ms": round(t_sw * 1e3, 4), "GB/s": round(b / t_sw / 1e9, 3)}
            x8 = cases.activations(m, K, cases.gen(3))
            t8, n8 = _time_cpu(lambda: tc.w8a16_ref(x8, wq8, sc8))
            b = N * K + 2 * N + 2 * m * K + 2 * m * N  # sweep.py:190-191
            rows[f"fp8_gate_up_M{m}"] = {"ms": round(t8 * 1e3, 3), "GB/s": round(b / t8 / 1e9, 3),
                                         "timed_calls": n8}
    finally:
        torch.set_num_threads(prev)
    return {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"config 0 through the reference CPU path restated in torch "
                      f"(oracle/torch_cpu.py: unpack + dequantize each call, fp32 matmul): median "
                      f"of {n} calls after warm-up, {sec * 1e3:.2f} ms/call; rows for config 1 and "
                      f"the FP8 path beside it; {time.perf_counter() - t_start:.1f} s in all",
            "threads": threads, "cpu_count": os.cpu_count(),
            "affinity": len(os.sched_getaffinity(0)), "cpu_model": _cpu_model(),
            "torch": torch.__version__, "rows": rows}


def e2e_leg(steps: int) -> dict:
    """Config 4, the metric's second half: batch-1 greedy decode of the random-init
    Qwen2.5-1.5B architecture (seed 4), 128-token prompt then `steps` decode steps, each step one
    hipGraph replay; fp16 library GEMMs against the swapped kernels. Every backend of one table
    runs the same lm_head: `head_gemv` sends the fp16 table (and the final norm) through this
    build's one-row GEMV on all backends, `head_torch` keeps the reference's norm then
    `F.linear(h, lm_head)` (model.py:250-253) on all backends. `ours_lm` quantizes the head
    instead. `decode_check` checks each timed generation teacher-forced against a reference
    runner on the same weights (kernels.e2e.run.decode_check). Reported beside the headline, not
    as `value`."""
    import gc

    import torch

    from kernels.e2e.run import run

    def table(res):
        b = res["backends"]
        return {"tok_s": {k: round(v["decode"]["tok_s"], 1) for k, v in b.items()},
                "ms_per_token": {k: round(v["decode"]["ms_per_token"], 3) for k, v in b.items()},
                "layers_only_ms": {k: round(v["layers_only_ms"], 3) for k, v in b.items()},
                "speedup_vs_fp16": {k: round(v["speedup_vs_fp16"], 3) for k, v in b.items()},
                "prefill_tok_s": {k: round(v["prefill"]["tok_s"], 1) for k, v in b.items()},
                "prefill_ms": {k: round(v["prefill"]["ms"], 3) for k, v in b.items()},
                "prefill_speedup_vs_fp16": {k: round(v["prefill_speedup_vs_fp16"], 3)
                                            for k, v in b.items()},
                "linear_bytes_per_token": {k: v["weights"]["linear_layers"] for k, v in b.items()},
                "decode_check": {k: {f: v["check"][f] for f in ("reference", "positions", "agree",
                                                              "max_margin", "beyond_tol")}
                                 for k, v in b.items() if "check" in v}}

    out = {"metric": "Qwen2.5-1.5B-arch batch-1 decode tok/s", "unit": "tok/s",
           "workload": "random-init Qwen2.5-1.5B architecture (seed 4), prompt 128, "
                       f"{steps} greedy steps, hipGraph per step, median of 3; prefill: the "
                       "128-token prompt's forward as one hipGraph, median of 5"}
    for head, backends in (("gemv", ["fp16", "ours", "ours_lm", "ours_fp8"]), ("torch", ["fp16", "ours"])):
        out[f"head_{head}"] = table(run({"backends": backends, "decode_steps": steps,
                                         "prompt_len": 128, "head": head}))
        gc.collect()
        torch.cuda.empty_cache()
    return out


def measured_traffic(kernel: str, kernel_config: str):
    """HBM bytes per launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary of this
    command (profiles/w4a16_m1_gate_up_traffic.md), or None when that summary was taken of
    another kernel or configuration than the one the library runs now."""
    path = REPO / "profiles" / "w4a16_m1_gate_up_traffic.md"
    try:
        text = path.read_text()
    except OSError:
        return None
    fields = {}
    for line in text.splitlines():
        key, sep, val = line.partition(":")
        if sep and key in ("traffic_bytes_per_launch", "kernel_config", "kernel"):
            fields[key] = val.strip()
    if fields.get("kernel_config") != kernel_config or fields.get("kernel") != kernel:
        return None
    return int(fields["traffic_bytes_per_launch"]) if "traffic_bytes_per_launch" in fields else None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000, help="minimum launches per timed sample")
    ap.add_argument("--warmup", type=int, default=500)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-e2e", action="store_true",
                    help="skip the config-4 decode leg (fp16 vs swapped tok/s)")
    ap.add_argument("--e2e-steps", type=int, default=256)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the W4A16 path would shard by output columns, each GPU its own tiles, with no "
              "exchange)",
              file=sys.stderr)
        return 2

    import torch

    from kernels.bench import cases
    from kernels.bench.harness import GraphTimer, n_copies
    from kernels.config import PEAK_GBPS
    from kernels.quant import quantize_rtn, weight_bytes
    from kernels.w4a16 import config_for, kernel_name, w4a16_matmul

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
    est_ms = timer.time_replays(warm_replays) / (warm_replays * per_replay)
    replays = max(math.ceil(args.steps / per_replay),
                  math.ceil(MIN_SAMPLE_MS / max(est_ms * per_replay, 1e-6)))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    samples = [timer.time_replays(replays) / (replays * per_replay) for _ in range(SAMPLES)]
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = statistics.median(samples)

    nbytes = weight_bytes(N, K, GS) + 2 * M * K + 2 * M * N  # sweep.py:167-169
    gbps = nbytes / (ms_per_step * 1e-3) / 1e9
    kcfg = config_for(M, N, K, GS)
    kname = kernel_name(M, N, K, GS)
    out = {
        "metric": METRIC,
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
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
        "timed": {"samples": SAMPLES, "launches_per_sample": replays * per_replay,
                  "warmup_launches": warm_replays * per_replay,
                  "sample_ms_per_launch": [round(v, 6) for v in samples],
                  "wall_s": round(wall, 3)},
        "pct_of_peak": round(100 * gbps / PEAK_GBPS, 2),
        "us_per_call": round(ms_per_step * 1e3, 3),
        "roofline": {"bound": "hbm", "achieved": round(gbps, 2), "peak": PEAK_GBPS,
                     "unit": "GB/s", "frac": round(gbps / PEAK_GBPS, 4),
                     "traffic": measured_traffic(kname, kcfg), "bytes_per_launch": nbytes,
                     "kernel": kname,
                     "timing": "HIP events on the graph-replay stream; median of 7 samples of "
                               ">= 50 ms of back-to-back launches"},
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
