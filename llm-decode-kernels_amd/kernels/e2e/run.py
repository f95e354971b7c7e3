"""End-to-end decode on one MI355X: the Qwen2.5-1.5B architecture, random-init (seed 4), fp16
library GEMMs vs this build's swapped kernels (config 4).

Measures per backend, same runner, hipGraphs on both sides (the reference's kernels/e2e/run.py):
- decode tokens/s at batch 1: a 128-token prompt of uniform random ids, then `decode_steps`
  greedy steps, each step one graph replay (forward + argmax + bookkeeping), median of 3 runs;
- the swapped layers alone: all 28 layers' projections, fused add+norms and the activation for
  one decode step, as one graph (`layers_only_ms`, run.py:166-201);
- the layer weight bytes each backend reads per token.

    python -m kernels.e2e.run [--backends fp16,ours] [--steps 256] [--prompt 128] [--json out]
"""

from __future__ import annotations

import argparse
import gc
import json
import statistics
import sys
import time

import torch

from kernels.bench.harness import capture
from kernels.e2e.model import QwenRunner, make_backend, random_qwen2


def _events():
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


class GraphDecoder:
    """One greedy decode step captured in a hipGraph (run.py:58-111)."""

    def __init__(self, runner: QwenRunner):
        self.r = runner
        dev = runner.embed.device
        self.tok = torch.zeros(1, 1, dtype=torch.long, device=dev)
        self.pos = torch.zeros(1, dtype=torch.long, device=dev)
        self.out = torch.zeros(runner.max_len, dtype=torch.long, device=dev)
        self.graph = None

    def _step(self):
        """forward + greedy bookkeeping. The argmax and the out/tok/pos updates run as one HIP
        launch (kernels.sample.greedy_step) on every backend: torch's vocabulary-sized argmax
        clears a semaphore with a memset node, which is not reliable under graph replay here."""
        from kernels.sample import greedy_step

        logits = self.r.forward(self.tok, self.pos)
        greedy_step(logits[:, -1], self.tok, self.pos, self.out)

    def prefill(self, ids: torch.Tensor) -> int:
        P = ids.shape[1]
        logits = self.r.forward(ids, torch.arange(P, device=ids.device))
        self.tok.copy_(logits[:, -1].argmax(-1).view(1, 1))
        self.pos.fill_(P)
        self.out.zero_()
        self.out[P - 1] = self.tok.view(-1)[0]  # position P-1 holds the first new token
        return P

    def capture(self, ids):
        """Eager warm-up first (the first library call per device allocates the split-K
        workspace), then capture on a side stream."""
        self.prefill(ids)
        self._step()
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(3):
                self._step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        self.prefill(ids)
        self.graph, _ = capture(self._step)
        torch.cuda.synchronize()

    def generate(self, ids, steps: int) -> tuple[list[int], float]:
        P = self.prefill(ids)
        torch.cuda.synchronize()
        start, end = _events()
        start.record()
        for _ in range(steps):
            self.graph.replay()
        end.record()
        torch.cuda.synchronize()
        tokens = self.out[P - 1: P - 1 + steps + 1].tolist()
        return tokens, start.elapsed_time(end) / 1e3


def decode_speed(runner, ids, steps: int, repeats: int = 3) -> dict:
    dec = GraphDecoder(runner)
    dec.capture(ids)
    rates, tokens = [], None
    for _ in range(repeats):
        tokens, sec = dec.generate(ids, steps)
        rates.append(steps / sec)
    del dec
    return {"tok_s": statistics.median(rates), "tok_s_min": min(rates), "tok_s_max": max(rates),
            "ms_per_token": 1e3 / statistics.median(rates), "steps": steps, "tokens": tokens}


def layers_only_ms(runner, M: int = 1) -> float:
    """Graph time of the swapped ops alone for one decode step (run.py:166-201): per layer the
    qkv, o, gate_up and down projections, two add+norms and the activation, through the
    backend's norm_linear/linear_norm_linear/act_linear (fused launches on the fused backends)."""
    be, eps = runner.backend, runner.eps
    dev = runner.embed.device
    H = runner.embed.shape[1]
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(1, M, H, device=dev, dtype=torch.float16, generator=g)
    res = torch.randn(1, M, H, device=dev, dtype=torch.float16, generator=g)
    nq, hd = runner.n_heads, runner.head_dim

    def step():
        h, r = x, res
        for L in runner.layers:
            qkv, r = be.norm_linear(h, L.ln1, eps, r, L.qkv)
            gate_up, r = be.linear_norm_linear(qkv[..., : nq * hd].contiguous(), L.o, r, L.ln2,
                                               eps, L.gate_up)
            h = be.act_linear(gate_up, L.down)

    for _ in range(3):
        step()
    torch.cuda.synchronize()
    graph, _ = capture(step)
    graph.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(7):
        start, end = _events()
        start.record()
        for _ in range(10):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end) / 10)
    del graph
    return statistics.median(times)


def run(params: dict) -> dict:
    backends = params.get("backends", ["fp16", "ours"])
    steps = int(params.get("decode_steps", 256))
    prompt_len = int(params.get("prompt_len", 128))
    seed = int(params.get("seed", 4))
    t0 = time.time()
    hf = random_qwen2(seed=seed)
    g = torch.Generator(device="cuda").manual_seed(seed)
    ids = torch.randint(0, hf.config.vocab_size, (1, prompt_len), device="cuda", generator=g)
    max_len = -(-(prompt_len + steps + 8) // 32) * 32  # the cache tiles hold 32 positions
    result = {"model": "Qwen2.5-1.5B architecture, random init (HF init, seed %d)" % seed,
              "prompt_len": prompt_len, "decode_steps": steps, "max_len": max_len,
              "backends": {}}
    for name in backends:
        print(f"[e2e] backend {name} ({time.time() - t0:.0f}s)", flush=True)
        runner = QwenRunner(hf, make_backend(name), max_len=max_len)
        r = {"weights": runner.weight_bytes()}
        r["decode"] = decode_speed(runner, ids, steps)
        r["layers_only_ms"] = layers_only_ms(runner)
        result["backends"][name] = r
        print(f"[e2e] {name}: {r['decode']['tok_s']:.1f} tok/s, layers only "
              f"{r['layers_only_ms']:.3f} ms ({time.time() - t0:.0f}s)", flush=True)
        del runner
        gc.collect()
        torch.cuda.empty_cache()
    if "fp16" in result["backends"]:
        base = result["backends"]["fp16"]
        for name, r in result["backends"].items():
            r["speedup_vs_fp16"] = r["decode"]["tok_s"] / base["decode"]["tok_s"]
            r["layers_speedup_vs_fp16"] = base["layers_only_ms"] / r["layers_only_ms"]
            toks, ref = r["decode"]["tokens"], base["decode"]["tokens"]
            r["first_token_divergence_vs_fp16"] = next(
                (i for i, (a, b) in enumerate(zip(toks, ref)) if a != b), len(toks))
    for r in result["backends"].values():
        r["decode"].pop("tokens", None)
    return result


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--backends", default="fp16,ours")
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--json", default=None)
    args = ap.parse_args(argv)
    res = run({"backends": args.backends.split(","), "decode_steps": args.steps,
               "prompt_len": args.prompt})
    text = json.dumps(res, indent=1)
    if args.json:
        with open(args.json, "w") as f:
            f.write(text)
    print(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
