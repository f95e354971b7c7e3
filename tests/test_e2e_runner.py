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


def test_decode_check_counts_agreement_and_margins():
    """decode_check (the teacher-forced check of bench's timed generations) on the CPU fp32
    runner: tokens of incremental greedy decoding agree at every position; a last token replaced
    by the least likely one is one disagreement, with the logit gap as its margin."""
    from kernels.e2e.run import decode_check

    model = _tiny_model(torch.float32, "cpu")
    runner = QwenRunner(model, make_backend("fp16"), max_len=64)
    ids = torch.randint(0, 512, (1, 8), generator=torch.Generator().manual_seed(2))
    logits = runner.forward(ids, torch.arange(8))
    toks = [int(logits[0, -1].argmax())]
    for t in range(8, 18):
        logits = runner.forward(torch.tensor([[toks[-1]]]), torch.tensor([t]))
        toks.append(int(logits[0, -1].argmax()))
    checker = QwenRunner(model, make_backend("fp16"), max_len=64)
    res = decode_check(checker, ids, toks)
    assert res["positions"] == 11 and res["agree"] == 11
    assert res["beyond_tol"] == 0 and res["max_margin"] == 0.0
    last = logits[0, -1]
    worst = int(last.argmin())
    bad = decode_check(checker, ids, toks[:-1] + [worst], tol=0.0)
    assert bad["agree"] == 10 and bad["beyond_tol"] == 1
    assert abs(bad["max_margin"] - float(last.max() - last.min())) < 1e-4


def test_check_reference_names():
    from kernels.e2e.run import check_reference

    assert check_reference("ours") == "w4_ref" and check_reference("ours_lm") == "w4_ref_lm"
    assert check_reference("ours_fp8") == "fp8_ref" and check_reference("fp16") == "fp16"
    assert make_backend("fp8_ref_lm").quant_lm_head


def test_lm_suffix_needs_quantized_backend():
    with pytest.raises(ValueError):
        make_backend("fp16_lm")


@pytest.mark.gpu
@pytest.mark.parametrize("ours", ["ours", "ours_cuda"])
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
        dec.step()
        eager.append(int(dec.tok.item()))
    assert P == 9 and toks == eager


def _qwen_heads_model(device, vocab=512, layers=2, intermediate=512):
    """Qwen2.5-1.5B attention geometry (12 query / 2 KV heads of 128) in a 2-layer model."""
    cfg = transformers.Qwen2Config(
        vocab_size=vocab, hidden_size=1536, intermediate_size=intermediate, num_hidden_layers=layers,
        num_attention_heads=12, num_key_value_heads=2, max_position_embeddings=1024,
        tie_word_embeddings=True, rms_norm_eps=1e-6, rope_theta=1e6,
    )
    torch.manual_seed(1)
    model = transformers.Qwen2ForCausalLM(cfg).to(device=device, dtype=torch.float16).eval()
    with torch.no_grad():
        for n, p in model.named_parameters():
            if n.endswith("bias") or "norm" in n:
                p.add_(0.05 * torch.randn_like(p))
    return model


@pytest.mark.gpu
@pytest.mark.parametrize("backend", ["fp16", "ours"])
def test_fused_decode_attention_matches_torch_path(backend):
    """Decode steps through the fused attention kernel (RoPE + KV write + GQA attention) against
    the torch ops of the same runner: close logits at every step and the same KV cache."""
    model = _qwen_heads_model("cuda")
    ref = QwenRunner(model, make_backend(backend), max_len=96, attention="torch")
    fused = QwenRunner(model, make_backend(backend), max_len=96, attention="fused")
    assert fused.fused_attention and not ref.fused_attention
    ids = torch.randint(0, 512, (1, 40), device="cuda")
    P = 30
    ref.forward(ids[:, :P], torch.arange(P, device="cuda"))
    fused.forward(ids[:, :P], torch.arange(P, device="cuda"))
    for t in range(P, 40):
        pos = torch.tensor([t], device="cuda")
        a = ref.forward(ids[:, t: t + 1], pos)
        b = fused.forward(ids[:, t: t + 1], pos)
        torch.testing.assert_close(b.float(), a.float(), atol=3e-2, rtol=3e-2)
    # Layer 0 sees identical inputs: v is copied as is; the roped k follows the same fp16
    # rounding steps, but torch's cos/sin and the kernel's differ in the last bits for angles up
    # to ~40 rad, which moves some results by an fp16 step (the kernel's RoPE is checked against
    # float64 in tests/test_gpu_attention.py). Later layers see hidden states that already differ
    # at fp16-ulp level through the attention outputs.
    from kernels.attention import k_from_tiles, v_from_tiles

    kf, kr = k_from_tiles(fused.k_cache)[..., :40, :].float(), k_from_tiles(ref.k_cache)[..., :40, :].float()
    vf, vr = v_from_tiles(fused.vt_cache)[..., :40, :], v_from_tiles(ref.vt_cache)[..., :40, :]
    assert (kf[0] - kr[0]).abs().max() < 1e-2
    assert torch.equal(vf[0], vr[0])
    torch.testing.assert_close(kf[1:], kr[1:], atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(vf[1:].float(), vr[1:].float(), atol=2e-2, rtol=2e-2)


@pytest.mark.gpu
@pytest.mark.parametrize("backend", ["ours", "ours_fp8"])
def test_attention_merged_in_o_projection_matches_merge_launch(backend):
    """The default decode step (the attention's four position ranges merged in the o
    projection's x staging, W4A16 or e4m3) against the same runner with the attention's own
    output (one range, no merge): close logits at every step across the range edges, identical
    KV caches."""
    model = _qwen_heads_model("cuda")
    merged = QwenRunner(model, make_backend(backend), max_len=416)
    plain = QwenRunner(model, make_backend(backend), max_len=416)
    assert merged.backend.merges_attention
    plain.merge_attention = False
    ids = torch.randint(0, 512, (1, 140), device="cuda")
    P = 120
    merged.forward(ids[:, :P], torch.arange(P, device="cuda"))
    plain.forward(ids[:, :P], torch.arange(P, device="cuda"))
    for t in range(P, 140):  # crosses the first range edge (128)
        pos = torch.tensor([t], device="cuda")
        a = plain.forward(ids[:, t: t + 1], pos)
        b = merged.forward(ids[:, t: t + 1], pos)
        torch.testing.assert_close(b.float(), a.float(), atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(merged.k_cache.float(), plain.k_cache.float(), atol=2e-2, rtol=2e-2)
    torch.testing.assert_close(merged.vt_cache.float(), plain.vt_cache.float(), atol=2e-2, rtol=2e-2)


@pytest.mark.gpu
@pytest.mark.parametrize("backend,T", [("ours", 128), ("ours_fp8", 256)])
def test_prompt_swiglu_in_gate_up_changes_no_logit(backend, T):
    """The prompt forward on `ours` and `ours_fp8` runs gate_up with SwiGLU in the prefill GEMM's
    epilogue (QwenRunner.fuse_prompt_act, kernels.fused.w4a16_matmul_swiglu and
    w8a16_matmul_swiglu): the prompt's logits at every
    position and the KV caches are bit-identical to the runner running gate_up then SwiGLU.
    Qwen2.5-1.5B's MLP (8960) at 128 prompt rows (int4) and 256 (e4m3), where the fused epilogue
    applies."""
    from kernels import _lib

    lib = _lib.load()
    applies = (lib.ldk_w4a16_matmul_swiglu_applies(T, 2 * 8960, 1536, 128) if backend == "ours"
               else lib.ldk_w8a16_matmul_swiglu_applies(T, 2 * 8960, 1536))
    assert applies == 1
    model = _qwen_heads_model("cuda", layers=2, intermediate=8960)
    fused = QwenRunner(model, make_backend(backend), max_len=416)
    plain = QwenRunner(model, make_backend(backend), max_len=416)
    assert fused.backend.fuses_prompt_act
    plain.fuse_prompt_act = False
    ids = torch.randint(0, 512, (1, T), device="cuda")
    pos = torch.arange(T, device="cuda")
    a = plain.forward(ids, pos, all_logits=True)
    b = fused.forward(ids, pos, all_logits=True)
    assert torch.equal(a, b)
    assert torch.equal(plain.k_cache, fused.k_cache) and torch.equal(plain.vt_cache, fused.vt_cache)


@pytest.mark.gpu
@pytest.mark.parametrize("backend", ["ours", "fp16"])
def test_warming_changes_no_logit(backend):
    """The fused attention's launch reading the next weights into the caches (QwenRunner.warm_set;
    the merged ranges on `ours`, the attention with its own output on `fp16`) leaves every decode
    step's logits and the KV caches bit-identical to the runner without it."""
    model = _qwen_heads_model("cuda")
    warm = QwenRunner(model, make_backend(backend), max_len=416)
    cold = QwenRunner(model, make_backend(backend), max_len=416)
    assert warm.backend.warms and warm.warm_weights and warm.warm_set(0)
    cold.warm_weights = False
    ids = torch.randint(0, 512, (1, 136), device="cuda")
    P = 124
    warm.forward(ids[:, :P], torch.arange(P, device="cuda"))
    cold.forward(ids[:, :P], torch.arange(P, device="cuda"))
    for t in range(P, 136):  # crosses the first range edge (128)
        pos = torch.tensor([t], device="cuda")
        assert torch.equal(warm.forward(ids[:, t: t + 1], pos), cold.forward(ids[:, t: t + 1], pos))
    assert torch.equal(warm.k_cache, cold.k_cache) and torch.equal(warm.vt_cache, cold.vt_cache)


@pytest.mark.gpu
def test_fused_attention_graph_decoder_matches_eager_steps():
    """The captured decode step with the fused attention replays exactly the eager steps."""
    from kernels.e2e.run import GraphDecoder

    model = _qwen_heads_model("cuda", vocab=151936)
    runner = QwenRunner(model, make_backend("ours"), max_len=128)
    assert runner.fused_attention
    ids = torch.randint(0, 151936, (1, 17), device="cuda")
    dec = GraphDecoder(runner)
    dec.capture(ids)
    toks, _ = dec.generate(ids, 24)
    P = dec.prefill(ids)
    eager = [int(dec.tok.item())]
    for _ in range(24):
        dec.step()
        eager.append(int(dec.tok.item()))
    assert P == 17 and toks == eager


def test_make_backend_names():
    for name in ("fp16", "w4_ref", "ours", "ours_cuda", "ours_fp8", "fp8_ref"):
        assert make_backend(name).name == name and not make_backend(name).quant_lm_head
    for name in ("w4_ref_lm", "ours_lm", "ours_cuda_lm", "ours_fp8_lm", "fp8_ref_lm"):
        be = make_backend(name)
        assert be.name == name and be.quant_lm_head and be.quantized
    with pytest.raises(KeyError):
        make_backend("ours_triton")


@pytest.mark.gpu
@pytest.mark.parametrize("backend", ["ours", "ours_lm", "ours_fp8", "fp16"])
def test_graph_generation_passes_decode_check(backend):
    """A GraphDecoder generation (what bench times) checked teacher-forced against the reference
    runner bench uses for it (dequantize + library GEMMs on the same weights; fp16: its own prompt
    path): no emitted token's logit is more than 5e-2 below the reference's argmax."""
    from kernels.e2e.run import GraphDecoder, check_reference, decode_check

    model = _tiny_model(torch.float16, "cuda")
    ids = torch.randint(0, 512, (1, 9), device="cuda", generator=torch.Generator("cuda").manual_seed(4))
    runner = QwenRunner(model, make_backend(backend), max_len=64)
    dec = GraphDecoder(runner)
    dec.capture(ids)
    toks, _ = dec.generate(ids, 24)
    ref = QwenRunner(model, make_backend(check_reference(backend)), max_len=64)
    res = decode_check(ref, ids, toks)
    assert res["positions"] == 25 and res["beyond_tol"] == 0, res


@pytest.mark.gpu
def test_fp8_ref_matches_ours_fp8():
    model = _tiny_model(torch.float16, "cuda")
    ids = torch.randint(0, 512, (1, 5), device="cuda")
    pos = torch.arange(5, device="cuda")
    ref = QwenRunner(model, make_backend("fp8_ref"), max_len=32).forward(ids, pos, all_logits=True)
    f8 = QwenRunner(model, make_backend("ours_fp8"), max_len=32).forward(ids, pos, all_logits=True)
    torch.testing.assert_close(f8.float(), ref.float(), atol=5e-2, rtol=5e-2)


@pytest.mark.gpu
@pytest.mark.parametrize("backend", ["fp16", "ours", "ours_fp8"])
def test_gemv_head_matches_torch_head(backend):
    """The runner's two lm_head paths (this build's one-row GEMV with the final norm in its
    launch, and the reference's norm then F.linear) give the same logits on every backend."""
    model = _qwen_heads_model("cuda", vocab=4096)
    ids = torch.randint(0, 4096, (1, 12), device="cuda")
    outs = {}
    for head in ("gemv", "torch"):
        r = QwenRunner(model, make_backend(backend), max_len=64, head=head)
        r.forward(ids[:, :11], torch.arange(11, device="cuda"))
        outs[head] = r.forward(ids[:, 11:], torch.tensor([11], device="cuda")).float()
    torch.testing.assert_close(outs["gemv"], outs["torch"], atol=1e-2, rtol=1e-2)


@pytest.mark.gpu
@pytest.mark.parametrize("backend", ["fp16", "ours", "ours_fp8"])
def test_prefill_speed_graph_matches_eager(backend):
    """The e2e prefill measurement (kernels.e2e.run.prefill_speed, the reference's
    run.py:142-162) replays a captured whole-prompt forward: its logits equal the eager
    forward's bit for bit (the same kernels on the same inputs), and it reports T tokens."""
    from kernels.bench.harness import capture
    from kernels.e2e.run import prefill_speed

    model = _tiny_model(torch.float16, "cuda")
    runner = QwenRunner(model, make_backend(backend), max_len=64)
    ids = torch.randint(0, 512, (1, 24), device="cuda", generator=torch.Generator("cuda").manual_seed(3))
    pos = torch.arange(24, device="cuda")
    eager = runner.forward(ids, pos).clone()
    graph, out = capture(lambda: runner.forward(ids, pos))
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, eager)
    res = prefill_speed(runner, ids)
    assert res["T"] == 24 and res["ms"] > 0 and res["tok_s"] > 0


@pytest.mark.gpu
@pytest.mark.parametrize("backend", ["fp16", "ours"])
@pytest.mark.parametrize("P", [2, 40, 130])
def test_fused_prefill_matches_torch_path(backend, P):
    """The prompt through ldk_prefill_attention (RoPE + KV write + causal GQA in two launches per
    layer) against the torch ops of the same runner: close logits for every prompt row, close
    KV caches (v of layer 0 identical), then decode steps that read the prompt's cache."""
    model = _qwen_heads_model("cuda")
    ref = QwenRunner(model, make_backend(backend), max_len=160, attention="torch")
    fused = QwenRunner(model, make_backend(backend), max_len=160, attention="fused")
    assert fused.fused_prefill and not ref.fused_prefill
    ids = torch.randint(0, 512, (1, P + 6), device="cuda")
    pos = torch.arange(P, device="cuda")
    a = ref.forward(ids[:, :P], pos, all_logits=True)
    b = fused.forward(ids[:, :P], pos, all_logits=True)
    torch.testing.assert_close(b.float(), a.float(), atol=3e-2, rtol=3e-2)
    from kernels.attention import k_from_tiles, v_from_tiles

    kf, kr = k_from_tiles(fused.k_cache)[..., :P, :].float(), k_from_tiles(ref.k_cache)[..., :P, :].float()
    vf, vr = v_from_tiles(fused.vt_cache)[..., :P, :], v_from_tiles(ref.vt_cache)[..., :P, :]
    assert (kf[0] - kr[0]).abs().max() < 1e-2
    assert torch.equal(vf[0], vr[0])
    torch.testing.assert_close(kf[1:], kr[1:], atol=2e-2, rtol=2e-2)
    for t in range(P, P + 6):
        step = torch.tensor([t], device="cuda")
        torch.testing.assert_close(fused.forward(ids[:, t: t + 1], step).float(),
                                   ref.forward(ids[:, t: t + 1], step).float(), atol=3e-2, rtol=3e-2)
