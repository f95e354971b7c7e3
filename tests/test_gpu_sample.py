"""The greedy decode step kernel (`ldk_greedy_step`, kernels.sample.greedy_step) against
torch.argmax, and inside captured hipGraphs replayed with eager work between the replays."""

import numpy as np
import pytest
import torch

from kernels.sample import greedy_step

pytestmark = pytest.mark.gpu


def _state(L=16, p=3):
    tok = torch.full((1, 1), -5, dtype=torch.int64, device="cuda")
    pos = torch.tensor([p], dtype=torch.int64, device="cuda")
    out = torch.full((L,), -7, dtype=torch.int64, device="cuda")
    return tok, pos, out


@pytest.mark.parametrize("V", [1, 7, 512, 4099, 151936, 151937])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_matches_torch_argmax(V, dtype):
    g = torch.Generator().manual_seed(V)
    logits = torch.randn(1, 1, V, generator=g).to(dtype)
    tok, pos, out = _state()
    greedy_step(logits.cuda(), tok, pos, out)
    want = int(logits.float().argmax())
    assert int(tok) == want and int(pos) == 4 and int(out[3]) == want
    assert torch.all(out[torch.arange(16, device="cuda") != 3] == -7)


def test_ties_take_the_lowest_index_and_nan_wins():
    x = torch.zeros(10000, dtype=torch.float16)
    x[[17, 9000, 4000]] = 3.0
    tok, pos, out = _state()
    greedy_step(x.cuda(), tok, pos, out)
    assert int(tok) == 17
    x[[5000, 6000]] = float("nan")
    greedy_step(x.cuda(), tok, pos, out)
    assert int(tok) == 5000 == int(torch.tensor(x.numpy()).argmax())
    assert int(pos) == 5 and int(out[4]) == 5000


def test_signed_zeros_tie_and_negative_nan_wins():
    x = torch.full((20000,), -1.0, dtype=torch.float32)
    x[11] = -0.0
    x[19000] = 0.0
    tok, pos, out = _state()
    greedy_step(x.cuda(), tok, pos, out)
    assert int(tok) == 11 == int(x.argmax())
    x[15000] = -float("nan")
    greedy_step(x.cuda(), tok, pos, out)
    assert int(tok) == 15000 == int(x.argmax())


def test_unaligned_row_takes_the_scalar_path():
    base = torch.randn(151937, dtype=torch.float16, device="cuda")
    row = base[1:]  # 2-byte offset: not 16-byte aligned
    tok, pos, out = _state()
    greedy_step(row, tok, pos, out)
    assert int(tok) == int(row.float().argmax())


def test_pos_outside_the_log_skips_the_write():
    tok, pos, out = _state(L=4, p=4)
    greedy_step(torch.arange(10, dtype=torch.float16, device="cuda"), tok, pos, out)
    assert int(tok) == 9 and int(pos) == 5 and torch.all(out == -7)


def test_replays_match_eager():
    """A captured lm_head GEMM + greedy step, replayed 20 times with new hidden states written
    eagerly between replays: every replay's token equals the eager argmax of the same logits."""
    g = torch.Generator(device="cuda").manual_seed(0)
    V, H = 151936, 1536
    W = (torch.randn(V, H, device="cuda", generator=g) * 0.02).half()
    h = torch.zeros(1, 1, H, dtype=torch.float16, device="cuda")
    tok, pos, out = _state(L=64, p=0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        greedy_step(torch.nn.functional.linear(h, W), tok, pos, out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        logits = torch.nn.functional.linear(h, W)
        greedy_step(logits, tok, pos, out)
    pos.zero_()
    for i in range(20):
        h.copy_(torch.randn(1, 1, H, device="cuda", generator=g).half())
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        want = int(torch.nn.functional.linear(h, W).float().argmax())
        assert int(tok) == want and int(out[i]) == want and int(pos) == i + 1, i
