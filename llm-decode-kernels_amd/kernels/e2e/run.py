"""End-to-end decode on one MI355X: the Qwen2.5-1.5B architecture, random-init (seed 4), fp16
library GEMMs vs this build's swapped kernels (config 4).

Measures per backend, same runner, hipGraphs on both sides (what the reference's
kernels/e2e/run.py measures on its GPUs):
- decode tokens/s at batch 1: a 128-token prompt of uniform random ids, then `decode_steps`
  greedy steps, each step one graph replay (forward + argmax + bookkeeping), median of 3 runs;
- the swapped layers alone: all 28 layers' projections, fused add+norms and the activation for
  one decode step, as one graph (`layers_only_ms`, the reference's run.py:166-201);
- prefill tokens/s: the whole 128-token prompt's forward as one graph, median of 5 replays
  (`prefill_speed`, the reference's run.py:142-162);
- the layer weight bytes each backend reads per token;
- a teacher-forced check of the timed generation (`decode_check`): one forward of the generated
  sequence through a reference runner (`CHECK_REFERENCE`) whose argmax at every position should
  be the emitted token.
Every backend runs the same lm_head (`--head gemv|torch`, kernels/e2e/model.py's QwenRunner).

    python -m kernels.e2e.run [--backends fp16,ours] [--steps 256] [--prompt 128] [--head gemv]
                              [--json out] [--no-check]
"""

from __future__ import annotations

import argparse
import gc
import json
import statistics
import sys
import time

import torch

from kernels.bench.harness import capture, replay_ms
from kernels.e2e.model import QwenRunner, make_backend, random_qwen2


class GraphDecoder:
    """Greedy batch-1 decoding, one hipGraph replay per token (the reference's run.py:58-122).

    The decode state lives on the device in one int64 buffer: [token, position, log of emitted
    tokens by position]. A step is the runner's forward on (token, position) followed by
    `kernels.sample.greedy_step` (argmax, log, advance) in one launch; the prompt's last logits go
    through the same launch, so the first new token is logged at position P - 1 like every
    later one at its own position."""

    def __init__(self, runner: QwenRunner):
        self.r = runner
        self.state = torch.zeros(2 + runner.max_len, dtype=torch.long, device=runner.embed.device)
        self.tok = self.state[:1].view(1, 1)
        self.pos = self.state[1:2]
        self.out = self.state[2:]
        self.graph = None

    def step(self):
        from kernels.sample import greedy_step

        greedy_step(self.r.forward(self.tok, self.pos), self.tok, self.pos, self.out)

    def prefill(self, ids: torch.Tensor) -> int:
        """Runs the prompt; leaves the first new token in `tok` and `out[P-1]`, position P."""
        from kernels.sample import greedy_step

        P = ids.shape[1]
        logits = self.r.forward(ids, torch.arange(P, device=ids.device))
        self.state.zero_()
        self.pos.fill_(P - 1)
        greedy_step(logits, self.tok, self.pos, self.out)
        return P

    def capture(self, ids: torch.Tensor, warmup: int = 3):
        """Eager steps on a side stream first (each library entry allocates its per-device
        workspace on its first call, which must not happen under capture), then the capture of
        one step from the state a fresh prefill leaves."""
        self.prefill(ids)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(warmup):
                self.step()
        torch.cuda.current_stream().wait_stream(side)
        self.prefill(ids)
        self.graph, _ = capture(self.step)
        torch.cuda.synchronize()

    def generate(self, ids: torch.Tensor, steps: int) -> tuple[list[int], float]:
        """Prefill, then `steps` replays. Returns the steps + 1 new tokens and the seconds the
        replays took (HIP events on the current stream)."""
        P = self.prefill(ids)
        torch.cuda.synchronize()
        ms = replay_ms(self.graph, steps)
        return self.out[P - 1: P + steps].tolist(), ms / 1e3


def decode_speed(runner, ids, steps: int, repeats: int = 3) -> dict:
    """Median decode rate over `repeats` generations of `steps` tokens after one prompt."""
    dec = GraphDecoder(runner)
    dec.capture(ids)
    runs = [dec.generate(ids, steps) for _ in range(repeats)]
    del dec
    rates = sorted(steps / sec for _, sec in runs)
    med = statistics.median(rates)
    return {"tok_s": med, "tok_s_min": rates[0], "tok_s_max": rates[-1],
            "ms_per_token": 1e3 / med, "steps": steps, "tokens": runs[-1][0]}


def prefill_speed(runner, ids: torch.Tensor, repeats: int = 5) -> dict:
    """The whole-prompt forward as one hipGraph (the reference's run.py:142-162): the T prompt
    tokens at positions 0..T-1 (KV cache written, last position's logits), two eager warm-up
    forwards, then the median of `repeats` single replays, HIP events on the replay stream."""
    T = ids.shape[1]
    pos = torch.arange(T, device=ids.device)
    for _ in range(2):
        runner.forward(ids, pos)
    torch.cuda.synchronize()
    graph, _ = capture(lambda: runner.forward(ids, pos))
    graph.replay()
    torch.cuda.synchronize()
    ms = statistics.median(replay_ms(graph, 1) for _ in range(repeats))
    del graph
    return {"T": T, "ms": ms, "tok_s": T / (ms * 1e-3)}


# The backend whose teacher-forced logits check each backend's timed generation: the same
# quantized weights through dequantize + library GEMMs (the reference's w4_ref role), and for
# fp16 the fp16 runner's own prompt path (library GEMMs and head, prompt attention) against its
# decode path (the one-row kernels).
CHECK_REFERENCE = {"fp16": "fp16", "w4_ref": "w4_ref", "ours": "w4_ref", "ours_cuda": "w4_ref",
                   "ours_fp8": "fp8_ref", "fp8_ref": "fp8_ref"}


def check_reference(name: str) -> str:
    """CHECK_REFERENCE for a backend name, `_lm` kept (the reference then quantizes its head too)."""
    base, lm = (name[:-3], "_lm") if name.endswith("_lm") else (name, "")
    return CHECK_REFERENCE[base] + lm


def decode_check(runner: QwenRunner, ids: torch.Tensor, tokens: list[int], tol: float = 5e-2) -> dict:
    """Teacher-forced check of a greedy generation: `tokens` are the steps + 1 tokens a decoder
    emitted after the prompt `ids` (the first predicted from the prompt's last position). One
    forward of `runner` over prompt + tokens[:-1] gives the logits at every position the decoder
    predicted from; its argmax should be the emitted token. Where it is not, `margin` is how far
    the emitted token's logit is below the argmax's (a near tie, flipped by the decode path's
    different summation order, has a margin within `tol`, the bound the runner tests hold the
    logits to, test_runner.py:48-85). Returns positions, agreements, the largest margin and how
    many margins exceed `tol`."""
    P = ids.shape[1]
    emitted = torch.tensor(tokens, dtype=torch.long, device=ids.device)
    seq = torch.cat([ids, emitted[None, :-1]], dim=1)
    with torch.no_grad():
        logits = runner.forward(seq, torch.arange(seq.shape[1], device=ids.device), all_logits=True)
    lg = logits[0, P - 1:].float()
    top = lg.argmax(-1)
    margin = lg.gather(1, top[:, None]) - lg.gather(1, emitted[:, None])
    return {"positions": len(tokens), "agree": int((top == emitted).sum()),
            "max_margin": float(margin.max()), "beyond_tol": int((margin > tol).sum()), "tol": tol}


def layers_only_ms(runner, M: int = 1, samples: int = 7, replays: int = 10) -> float:
    """Graph time of the swapped ops alone for one decode step (the reference's run.py:166-201):
    per layer the qkv, o, gate_up and down projections, two add+norms and the activation,
    through the backend's norm_linear/linear_norm_linear/act_linear (fused launches on the fused
    backends). Median over `samples` of `replays` back-to-back replays."""
    be, eps = runner.backend, runner.eps
    dev = runner.embed.device
    H = runner.embed.shape[1]
    g = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(1, M, H, device=dev, dtype=torch.float16, generator=g)
    res = torch.randn(1, M, H, device=dev, dtype=torch.float16, generator=g)
    q_width = runner.n_heads * runner.head_dim

    def body():
        h, r = x, res
        for L in runner.layers:
            qkv, r = be.norm_linear(h, L.ln1, eps, r, L.qkv)
            gate_up, r = be.linear_norm_linear(qkv[..., :q_width].contiguous(), L.o, r, L.ln2,
                                               eps, L.gate_up)
            h = be.act_linear(gate_up, L.down)

    for _ in range(3):
        body()
    torch.cuda.synchronize()
    graph, _ = capture(body)
    graph.replay()
    ms = statistics.median(replay_ms(graph, replays) / replays for _ in range(samples))
    del graph
    return ms


def run(params: dict) -> dict:
    backends = params.get("backends", ["fp16", "ours"])
    steps = int(params.get("decode_steps", 256))
    prompt_len = int(params.get("prompt_len", 128))
    seed = int(params.get("seed", 4))
    head = params.get("head", "gemv")
    check = bool(params.get("check", True))
    t0 = time.time()
    hf = random_qwen2(seed=seed)
    g = torch.Generator(device="cuda").manual_seed(seed)
    ids = torch.randint(0, hf.config.vocab_size, (1, prompt_len), device="cuda", generator=g)
    max_len = -(-(prompt_len + steps + 8) // 32) * 32  # the cache tiles hold 32 positions
    result = {"model": "Qwen2.5-1.5B architecture, random init (HF init, seed %d)" % seed,
              "prompt_len": prompt_len, "decode_steps": steps, "max_len": max_len,
              "head": head, "backends": {}}
    for name in backends:
        print(f"[e2e] backend {name}, head {head} ({time.time() - t0:.0f}s)", file=sys.stderr, flush=True)
        runner = QwenRunner(hf, make_backend(name), max_len=max_len, head=head)
        r = {"weights": runner.weight_bytes()}
        r["decode"] = decode_speed(runner, ids, steps)
        r["layers_only_ms"] = layers_only_ms(runner)
        r["prefill"] = prefill_speed(runner, ids)
        result["backends"][name] = r
        print(f"[e2e] {name}: {r['decode']['tok_s']:.1f} tok/s, layers only "
              f"{r['layers_only_ms']:.3f} ms, prefill {r['prefill']['T']} tokens "
              f"{r['prefill']['ms']:.3f} ms ({r['prefill']['tok_s']:.0f} tok/s) "
              f"({time.time() - t0:.0f}s)", file=sys.stderr, flush=True)
        del runner
        gc.collect()
        torch.cuda.empty_cache()
        if check:
            ref_name = check_reference(name)
            ref = QwenRunner(hf, make_backend(ref_name), max_len=max_len, head=head)
            r["check"] = {"reference": ref_name, **decode_check(ref, ids, r["decode"]["tokens"])}
            c = r["check"]
            print(f"[e2e] {name} against {ref_name}, teacher-forced: {c['agree']}/{c['positions']} "
                  f"tokens agree, largest margin {c['max_margin']:.4f}, {c['beyond_tol']} beyond "
                  f"{c['tol']} ({time.time() - t0:.0f}s)", file=sys.stderr, flush=True)
            del ref
            gc.collect()
            torch.cuda.empty_cache()
    if "fp16" in result["backends"]:
        base = result["backends"]["fp16"]
        for name, r in result["backends"].items():
            r["speedup_vs_fp16"] = r["decode"]["tok_s"] / base["decode"]["tok_s"]
            r["prefill_speedup_vs_fp16"] = r["prefill"]["tok_s"] / base["prefill"]["tok_s"]
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
    ap.add_argument("--head", default="gemv", choices=QwenRunner.HEADS)
    ap.add_argument("--json", default=None)
    ap.add_argument("--no-check", action="store_true",
                    help="skip the teacher-forced check of each timed generation")
    args = ap.parse_args(argv)
    res = run({"backends": args.backends.split(","), "decode_steps": args.steps,
               "prompt_len": args.prompt, "head": args.head, "check": not args.no_check})
    text = json.dumps(res, indent=1)
    if args.json:
        with open(args.json, "w") as f:
            f.write(text)
    print(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
