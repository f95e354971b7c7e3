"""The kernel sweep's aggregation over repeated sweeps (host logic, no GPU): median per row,
min/max, and the >10% spread flag of the reference's kernels/bench/sweep.py:229-254."""

from kernels.bench.sweep import _row, aggregate


def _sweep(us_a, us_b):
    return [_row("w4a16", "gate_up 17920x1536", 1, us_a * 1e-3, 13_762_560),
            {**_row("w4a16 gemm", "qkv 2048x1536", 2048, us_b * 1e-3, 10_000_000),
             "flops": 2 * 2048 * 2048 * 1536, "config": "w4a16_gemm_kernel<4, 4, 2, 2>"}]


def test_median_min_max_and_spread_flag():
    agg = aggregate([_sweep(5.0, 19.0), _sweep(5.2, 25.0), _sweep(5.1, 19.5)])
    a, b = agg
    assert a["us"] == 5.1 and a["us_min"] == 5.0 and a["us_max"] == 5.2 and a["sweeps"] == 3
    assert abs(a["spread_pct"] - 100 * 0.2 / 5.1) < 0.01 and not a["flag_spread"]
    assert abs(a["gbps"] - 13_762_560 / 5.1e-6 / 1e9) < 0.1
    assert b["us"] == 19.5 and b["flag_spread"] and b["spread_pct"] > 10
    assert b["config"] == "w4a16_gemm_kernel<4, 4, 2, 2>"
    assert abs(b["tflops"] - 2 * 2048 * 2048 * 1536 / 19.5e-6 / 1e12) < 0.1


def test_single_sweep_has_no_spread():
    (a, _), = [aggregate([_sweep(5.0, 19.0)])]
    assert a["spread_pct"] == 0 and not a["flag_spread"] and a["sweeps"] == 1
