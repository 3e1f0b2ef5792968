"""Token sampling (qwen3-1.7b/kernels.py:1286-1370) on the GPU against the oracle: greedy argmax
with the first-index tie-break over Qwen3's 151,936-entry vocabulary (ties inside one 8,192-entry
block and across blocks, all-equal and -inf rows, bf16 and fp32 logits, unaligned rows),
Gumbel-max sampling with Triton's Philox stream at tau > 0, the seed increment (also for an
empty batch) and graph replays drawing successive seeds."""

import numpy as np
import pytest
import torch

from helpers import say
from oracle import sampling as osm

VOCAB = 151_936


def _seed(dev, s):
    return torch.tensor([s], dtype=torch.int64, device=dev)


def _check(ie, logits, tau, s0, what):
    seed = _seed(logits.device, s0)
    tok = ie.sample(logits, tau, seed)
    torch.cuda.synchronize()
    ref, nxt = osm.sample(logits.float().cpu().numpy(), tau, s0)
    assert tok.dtype == torch.int64 and tok.shape == (logits.shape[0], 1)
    got = tok.cpu().numpy()
    bad = np.nonzero(got[:, 0] != ref[:, 0])[0]
    assert bad.size == 0, f"{what}: rows {bad[:8].tolist()} differ: {got[bad[:8], 0]} vs {ref[bad[:8], 0]}"
    assert int(seed.item()) == nxt
    say(f"{what}: {logits.shape[0]} rows match")


@pytest.mark.gpu
def test_greedy_qwen_vocab_with_ties(ie, dev):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(32, VOCAB, generator=g) * 3
    x[1, [100, 5000]] = 20.0  # tie inside block 0: 100 wins
    x[2, [9000, 70000]] = 20.0  # tie across blocks: 9000 wins
    x[3, :] = 1.5  # all equal: index 0
    x[4, :] = -float("inf")
    x[4, VOCAB - 1] = -1e30  # the last index
    x[5, VOCAB - 1] = 50.0
    x[6, :] = -float("inf")  # all -inf: index 0 (the reference's first index)
    _check(ie, x.bfloat16().to(dev), 0.0, 7, "greedy bf16")
    _check(ie, x.to(dev), 0.0, 7, "greedy fp32")


@pytest.mark.gpu
def test_greedy_unaligned_rows(ie, dev):
    # a vocabulary that is not a multiple of 8 and rows that are views of a wider buffer
    g = torch.Generator().manual_seed(1)
    wide = torch.randn(9, 1013, generator=g).bfloat16().to(dev)
    _check(ie, wide[:, 3:1004], 0.0, 0, "greedy strided bf16")
    _check(ie, wide.float()[:, 1:1002], 0.0, 0, "greedy strided fp32")


@pytest.mark.gpu
@pytest.mark.parametrize("tau,V", [(1.0, 5000), (0.6, VOCAB)])
def test_gumbel_matches_oracle(ie, dev, tau, V):
    g = torch.Generator().manual_seed(2)
    x = (torch.randn(16, V, generator=g) * 2).bfloat16().to(dev)
    for s0 in (0, 123456789, 2 ** 40 + 3):
        _check(ie, x, tau, s0, f"gumbel tau={tau} V={V} seed={s0}")


@pytest.mark.gpu
def test_empty_batch_still_advances_seed(ie, dev):
    seed = _seed(dev, 5)
    tok = ie.sample(torch.empty(0, VOCAB, dtype=torch.bfloat16, device=dev), 0.7, seed)
    torch.cuda.synchronize()
    assert tok.shape == (0, 1) and int(seed.item()) == 6


@pytest.mark.gpu
def test_graph_replays_draw_successive_seeds(ie, dev):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(8, 3000, generator=g).bfloat16().to(dev)
    seed = _seed(dev, 0)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ie.sample(x, 1.0, seed)  # warm-up (executes)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ie.sample(x, 1.0, seed)
    torch.cuda.synchronize()
    seed.fill_(1000)
    xs = x.float().cpu().numpy()
    for r in range(3):
        graph.replay()
        torch.cuda.synchronize()
        ref, _ = osm.sample(xs, 1.0, 1000 + r)
        assert np.array_equal(out.cpu().numpy(), ref), f"replay {r}"
        say(f"graph replay {r}: matches seed {1000 + r}")
    assert int(seed.item()) == 1003
