"""Config 4 at full size: the random-init Qwen2.5-1.5B architecture (28 layers, hidden 1536,
12/2 heads of 128, intermediate 8960, vocabulary 151936, seed 4), not a shrunken copy.

- `ours` and `ours_lm` against `w4_ref` and `w4_ref_lm` (the same int4 weights dequantized then
  library GEMMs): the prompt's logits and several decode steps' logits within the reference's
  5e-2 (tests/test_runner.py:48-70 of the reference, there on a 2-layer model);
- the captured decode step against eager steps for 32 tokens at max_len 416 (the hipGraph path
  that bench.py times), token for token.
"""

import gc

import pytest
import torch

transformers = pytest.importorskip("transformers")

from kernels.e2e.model import QwenRunner, make_backend, random_qwen2  # noqa: E402

pytestmark = pytest.mark.gpu

PROMPT, STEPS, MAX_LEN = 128, 6, 416


@pytest.fixture(scope="module")
def model():
    print("[config4] building the random-init Qwen2.5-1.5B model (seed 4)", flush=True)
    m = random_qwen2(seed=4)
    yield m
    del m
    gc.collect()
    torch.cuda.empty_cache()


@pytest.fixture(scope="module")
def prompt(model):
    g = torch.Generator(device="cuda").manual_seed(4)
    return torch.randint(0, model.config.vocab_size, (1, PROMPT), device="cuda", generator=g)


def _lockstep(ref: QwenRunner, ours: QwenRunner, ids):
    """Prompt logits of both runners, then STEPS decode steps fed the reference's greedy token,
    so both see the same inputs at every step."""
    P = ids.shape[1]
    pos = torch.arange(P, device="cuda")
    pairs = [(ref.forward(ids, pos, all_logits=True), ours.forward(ids, pos, all_logits=True))]
    tok = pairs[0][0][:, -1:].argmax(-1)
    for t in range(P, P + STEPS):
        p = torch.tensor([t], device="cuda")
        a, b = ref.forward(tok, p), ours.forward(tok, p)
        pairs.append((a, b))
        tok = a[:, -1:].argmax(-1)
    return pairs


@pytest.mark.parametrize("ours,ref", [("ours", "w4_ref"), ("ours_lm", "w4_ref_lm")])
def test_full_size_logits_match_dequantized_reference(model, prompt, ours, ref):
    print(f"[config4] {ours} vs {ref}: prompt {PROMPT}, {STEPS} decode steps", flush=True)
    r_ref = QwenRunner(model, make_backend(ref), max_len=MAX_LEN)
    r_ours = QwenRunner(model, make_backend(ours), max_len=MAX_LEN)
    assert len(r_ours.layers) == 28 and r_ours.lm_head.shape == (151936, 1536)
    worst = 0.0
    for i, (a, b) in enumerate(_lockstep(r_ref, r_ours, prompt)):
        assert torch.isfinite(b).all()
        torch.testing.assert_close(b.float(), a.float(), atol=5e-2, rtol=5e-2,
                                   msg=lambda m, i=i: f"step {i}: {m}")
        worst = max(worst, float((b.float() - a.float()).abs().max()))
    print(f"[config4] {ours}: worst |logit difference| {worst:.4f}", flush=True)
    del r_ref, r_ours
    gc.collect()
    torch.cuda.empty_cache()


def test_full_size_graph_decode_matches_eager(model, prompt):
    from kernels.e2e.run import GraphDecoder

    print("[config4] ours: 32 captured decode steps vs eager, max_len 416", flush=True)
    runner = QwenRunner(model, make_backend("ours"), max_len=MAX_LEN)
    assert runner.fused_attention
    dec = GraphDecoder(runner)
    dec.capture(prompt)
    graph_tokens, _ = dec.generate(prompt, 32)
    P = dec.prefill(prompt)
    eager = [int(dec.tok.item())]
    for _ in range(32):
        dec.step()
        eager.append(int(dec.tok.item()))
    assert P == PROMPT and graph_tokens == eager
    assert int(dec.pos.item()) == PROMPT + 32
    del dec, runner
    gc.collect()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("P", [40, 200])
def test_full_size_prompt_lengths_match_dequantized_reference(model, P):
    """Other prompt lengths at full size run other prefill plans (40 rows: 16-row blocks on qkv, o
    and down, down in 3 K splits; 200 rows: 32-row blocks on qkv and o, 128-column tiles in 3 K
    splits on down):
    every prompt row's logits of `ours` against `w4_ref` within the reference's 5e-2."""
    print(f"[config4] ours vs w4_ref: prompt {P}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(40 + P)
    ids = torch.randint(0, model.config.vocab_size, (1, P), device="cuda", generator=g)
    pos = torch.arange(P, device="cuda")
    r_ref = QwenRunner(model, make_backend("w4_ref"), max_len=MAX_LEN)
    r_ours = QwenRunner(model, make_backend("ours"), max_len=MAX_LEN)
    a = r_ref.forward(ids, pos, all_logits=True)
    b = r_ours.forward(ids, pos, all_logits=True)
    assert torch.isfinite(b).all()
    torch.testing.assert_close(b.float(), a.float(), atol=5e-2, rtol=5e-2)
    del r_ref, r_ours
    gc.collect()
    torch.cuda.empty_cache()
