"""The e2e runner on a tiny random Qwen2 (the reference's tests/test_runner.py cases).

CPU tier: the fp32 runner against Hugging Face's own Qwen2 forward (atol 1e-4), and prefill +
incremental decode against one full forward (the static KV cache works). GPU tier: the swapped
kernels against the dequantize-then-GEMM reference on the same int4 weights, and FP8 against
fp16 (both within 5e-2, test_runner.py:48-85)."""

import pytest
import torch

transformers = pytest.importorskip("transformers")

from kernels.e2e.model import QwenRunner, make_backend  # noqa: E402


def _tiny_model(dtype, device, vocab=512):
    cfg = transformers.Qwen2Config(
        vocab_size=vocab, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
        num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=256,
        tie_word_embeddings=True, rms_norm_eps=1e-6,
    )
    torch.manual_seed(0)
    model = transformers.Qwen2ForCausalLM(cfg).to(device=device, dtype=dtype).eval()
    # HF initialises biases and norm weights to 0 and 1; perturb them so both paths are exercised
    with torch.no_grad():
        for n, p in model.named_parameters():
            if n.endswith("bias") or "norm" in n:
                p.add_(0.05 * torch.randn_like(p))
    return model


def test_runner_matches_hf_fp32():
    model = _tiny_model(torch.float32, "cpu")
    ids = torch.randint(0, 512, (1, 12))
    with torch.no_grad():
        ref = model(ids).logits
    runner = QwenRunner(model, make_backend("fp16"), max_len=64)  # torch ops on CPU, fp32
    out = runner.forward(ids, torch.arange(12), all_logits=True)
    torch.testing.assert_close(out, ref, atol=1e-4, rtol=1e-4)


def test_runner_incremental_decode_matches_full():
    """Prefill 8 tokens, then decode 4 one at a time == one 12-token forward."""
    model = _tiny_model(torch.float32, "cpu")
    ids = torch.randint(0, 512, (1, 12))
    runner = QwenRunner(model, make_backend("fp16"), max_len=64)
    full = runner.forward(ids, torch.arange(12), all_logits=True)
    runner.forward(ids[:, :8], torch.arange(8))
    for t in range(8, 12):
        step = runner.forward(ids[:, t: t + 1], torch.tensor([t]))
        torch.testing.assert_close(step[0, -1], full[0, t], atol=1e-4, rtol=1e-4)


def test_lm_suffix_needs_quantized_backend():
    with pytest.raises(ValueError):
        make_backend("fp16_lm")


@pytest.mark.gpu
@pytest.mark.parametrize("ours", ["ours", "ours_hip"])
def test_ours_matches_w4_reference(ours):
    model = _tiny_model(torch.float16, "cuda")
    ids = torch.randint(0, 512, (1, 5), device="cuda")
    pos = torch.arange(5, device="cuda")
    ref = QwenRunner(model, make_backend("w4_ref"), max_len=32).forward(ids, pos, all_logits=True)
    out = QwenRunner(model, make_backend(ours), max_len=32).forward(ids, pos, all_logits=True)
    torch.testing.assert_close(out.float(), ref.float(), atol=5e-2, rtol=5e-2)


@pytest.mark.gpu
def test_ours_lm_matches_w4_ref_lm():
    model = _tiny_model(torch.float16, "cuda")
    ids = torch.randint(0, 512, (1, 5), device="cuda")
    pos = torch.arange(5, device="cuda")
    ref_r = QwenRunner(model, make_backend("w4_ref_lm"), max_len=32)
    ours_r = QwenRunner(model, make_backend("ours_lm"), max_len=32)
    assert ours_r.weight_bytes()["lm_head_quantized"]
    ref = ref_r.forward(ids, pos, all_logits=True)
    ours = ours_r.forward(ids, pos, all_logits=True)
    torch.testing.assert_close(ours.float(), ref.float(), atol=5e-2, rtol=5e-2)
    plain = QwenRunner(model, make_backend("w4_ref"), max_len=32).forward(ids, pos, all_logits=True)
    assert not torch.equal(ref, plain)


@pytest.mark.gpu
def test_ours_fp8_close_to_fp16():
    model = _tiny_model(torch.float16, "cuda")
    ids = torch.randint(0, 512, (1, 5), device="cuda")
    pos = torch.arange(5, device="cuda")
    ref = QwenRunner(model, make_backend("fp16"), max_len=32).forward(ids, pos, all_logits=True)
    f8 = QwenRunner(model, make_backend("ours_fp8"), max_len=32).forward(ids, pos, all_logits=True)
    torch.testing.assert_close(f8.float(), ref.float(), atol=5e-2, rtol=5e-2)


@pytest.mark.gpu
@pytest.mark.parametrize("vocab", [512, 151936])
def test_graph_decoder_matches_eager_steps(vocab):
    """The captured decode step replays exactly the eager greedy steps (ours backend), also at
    the real vocabulary size."""
    from kernels.e2e.run import GraphDecoder

    model = _tiny_model(torch.float16, "cuda", vocab)
    runner = QwenRunner(model, make_backend("ours"), max_len=64)
    ids = torch.randint(0, vocab, (1, 9), device="cuda")
    dec = GraphDecoder(runner)
    dec.capture(ids)
    toks, _ = dec.generate(ids, 12)
    P = dec.prefill(ids)
    eager = [int(dec.tok.item())]
    for _ in range(12):
        dec._step()
        eager.append(int(dec.tok.item()))
    assert P == 9 and toks == eager
