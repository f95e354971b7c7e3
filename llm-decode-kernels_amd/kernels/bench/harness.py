"""hipGraph timing with rotating buffers, re-done for MI355X from the reference's method
(kernels/bench/harness.py:18-174, frozen in docs/DECISIONS.md:27-52 of the reference):

- Rotating input copies so that every call reads from HBM: the working set is sized to 4x the
  256 MB Infinity Cache (MALL), not to torch's per-XCD L2 figure, which on MI355X is 16x too
  small to defeat caching.
- One graph of one call per copy, replayed until >= MIN_MS; the median of MEASUREMENTS samples.
  Every call writes its own output buffer (kept alive across the capture).
- HIP events are recorded on the stream the graph is replayed on.
"""

from __future__ import annotations

import contextlib
import gc
import math
import statistics
from collections.abc import Callable

import torch

WARMUP_CALLS = 3
MEASUREMENTS = 7
MIN_MS = 50.0
MALL_BYTES = 256 * 2**20
MEMORY_BUDGET = 8 * 2**30  # bytes of rotating copies per case (of 288 GB HBM)


def tensor_bytes(obj) -> int:
    """Bytes of every tensor in a (nested) list/tuple/dict."""
    from torch.utils._pytree import tree_leaves

    return sum(t.nbytes for t in tree_leaves(obj) if isinstance(t, torch.Tensor))


def n_copies(bytes_per_set: int, cache_bytes: int = MALL_BYTES, cap: int = 1024) -> int:
    """Copies needed for a working set of 4x the cache, within the memory budget."""
    want = math.ceil(4 * cache_bytes / max(bytes_per_set, 1))
    budget = max(2, MEMORY_BUDGET // max(bytes_per_set, 1))
    return int(min(max(want, 2), budget, cap))


@contextlib.contextmanager
def _gc_paused():
    """Python's collector may free a tensor whose memory a capture is recording into."""
    was = gc.isenabled()
    gc.collect()
    gc.disable()
    try:
        yield
    finally:
        if was:
            gc.enable()


def capture(body: Callable):
    """(graph, body's result) for one capture of body() on a side stream."""
    graph = torch.cuda.CUDAGraph()
    with _gc_paused(), torch.cuda.graph(graph, capture_error_mode="thread_local"):
        result = body()
    return graph, result


def replay_ms(graph, replays: int, stream=None) -> float:
    """ms of `replays` back-to-back replays of `graph`, HIP events on `stream` (default: the
    current stream), which is where the replays run."""
    stream = stream or torch.cuda.current_stream()
    start, end = (torch.cuda.Event(enable_timing=True) for _ in range(2))
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(replays):
            graph.replay()
        end.record(stream)
    end.synchronize()
    return start.elapsed_time(end)


class GraphTimer:
    """A captured graph of fn(*set) for every rotating set, replayed on its own stream."""

    def __init__(self, fn: Callable, sets: list):
        self.sets = sets
        self.stream = torch.cuda.Stream()
        self.stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(self.stream):
            for args in sets[:WARMUP_CALLS]:
                fn(*args)
        torch.cuda.current_stream().wait_stream(self.stream)
        torch.cuda.synchronize()
        self.graph, self.outs = capture(lambda: [fn(*args) for args in sets])
        self.graph.replay()
        torch.cuda.synchronize()

    @property
    def calls_per_replay(self) -> int:
        return len(self.sets)

    def time_replays(self, replays: int) -> float:
        """Total ms of `replays` back-to-back replays, HIP events on the replay stream."""
        return replay_ms(self.graph, replays, self.stream)

    def median_ms_per_call(self) -> float:
        first = self.time_replays(1)
        replays = max(1, math.ceil(MIN_MS / max(first, 1e-3)))
        samples = [self.time_replays(replays) / (replays * len(self.sets))
                   for _ in range(MEASUREMENTS)]
        return statistics.median(samples)

    def close(self):
        del self.graph, self.outs
        torch.cuda.synchronize()


def metrics(ms: float, bytes_moved: int, flops: int = 0, peak_gbps: float = 8000.0,
            peak_tflops: float = 2500.0) -> dict:
    """GB/s, % of HBM peak, TFLOP/s and intensity for one call (harness.py:163-174)."""
    s = ms * 1e-3
    gbps = bytes_moved / s / 1e9
    tflops = flops / s / 1e12 if flops else 0.0
    return {"us": ms * 1e3, "gbps": gbps, "pct_peak_bw": 100 * gbps / peak_gbps,
            "tflops": tflops, "pct_peak_flops": 100 * tflops / peak_tflops if flops else 0.0,
            "intensity": flops / bytes_moved if flops else 0.0}
