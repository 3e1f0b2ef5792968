"""Whole decode step of a Qwen3-shaped model (2 layers, small vocab) with the int8-KV attention
kernels, captured as a hipGraph: replays are bit-identical to eager steps, also after the
step's inputs change in place (qwen3-1.7b/engine.py:376-470)."""

import importlib

import pytest
import torch

from helpers import say

pytestmark = pytest.mark.gpu


def test_decode_step_graph_bitwise(ie, dev):
    ds = importlib.import_module("inference-engine_amd.decode_step")
    shape = ds.Qwen3Shape(layers=2, vocab=4096)
    say("decode step graph: 2 layers, B=8, ctx ~ U[16, 512)")
    step = ds.make_decode_step(batch=8, ctx_lo=16, ctx_hi=512, shape=shape, device=dev, seed=3)
    eager = step.forward().clone()
    assert eager.shape == (8, 1) and eager.dtype == torch.int64
    graph, out = step.capture()
    junk = torch.randn(256, 256, device=dev)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs from the eager step"
        junk = junk @ junk.T / 256
        torch.cuda.synchronize()
    # the next step: every sequence one token longer, new input tokens
    step.cached_lens.add_(1)
    step.ids.copy_(out.view(-1))
    graph.replay()
    torch.cuda.synchronize()
    nxt = out.clone()
    assert torch.equal(nxt, step.forward()), "replay after input change differs from eager"


def test_decode_step_attention_matches_parts(ie, dev):
    """The step's attention sub-block equals the same kernels called one by one."""
    ds = importlib.import_module("inference-engine_amd.decode_step")
    shape = ds.Qwen3Shape(layers=1, vocab=1024)
    step = ds.make_decode_step(batch=4, ctx_lo=64, ctx_hi=256, shape=shape, device=dev, seed=5)
    cos, sin = step._rope()
    x = torch.randn(4, shape.model_dim, device=dev).bfloat16()
    got = step.attention(0, x, cos, sin)  # the second call below rewrites the same cache column
    lw = step.layers[0]
    qkv = ie.kernels.linear(x, lw.qkv)  # the step's projection (tuned: skinny or library)
    q, k, v = qkv.split([2048, 1024, 1024], dim=-1)
    qo = ie.fused_rope_kv_decode(q.view(4, 16, 128), k.view(4, 8, 128), v.view(4, 8, 128),
                                 lw.q_norm, lw.k_norm, cos, sin, step.slot_ids, step.caches[0],
                                 step.cached_lens, step.num_decoding, 1e-6)
    o = ie.decode_attention(qo, step.caches[0], step.cached_lens, step.slot_ids,
                            step.num_decoding, 128 ** -0.5)
    want = ie.kernels.linear(o.view(4, -1), lw.o_proj)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
