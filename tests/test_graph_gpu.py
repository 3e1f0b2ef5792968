"""hipGraph capture of the decode step (torch.cuda.graph is hipGraph on ROCm): replays are
bit-identical to eager execution, also after the step's inputs change in place
(qwen3-1.7b/engine.py:432-470 capture/replay pattern)."""

import pytest
import torch

from helpers import say

pytestmark = pytest.mark.gpu


def _make_step(ie, dev, layers=3, B=8, pool=12, max_len=1024, seed=0):
    g = torch.Generator(device=dev).manual_seed(seed)
    caches = []
    for _ in range(layers):
        c = ie.make_layer_cache(pool, 8, max_len, 128, device=dev)
        c.k.copy_(torch.randint(-127, 128, c.k.shape, generator=g, device=dev, dtype=torch.int8))
        c.v.copy_(torch.randint(-127, 128, c.v.shape, generator=g, device=dev, dtype=torch.int8))
        c.k_scale.copy_(torch.rand(c.k_scale.shape, generator=g, device=dev) * 0.05)
        c.v_scale.copy_(torch.rand(c.v_scale.shape, generator=g, device=dev) * 0.05)
        caches.append(c)
    static = dict(
        qkv=torch.randn(layers, B, 32 * 128, generator=g, device=dev).bfloat16(),
        qw=torch.ones(128, device=dev, dtype=torch.bfloat16),
        kw=torch.ones(128, device=dev, dtype=torch.bfloat16),
        cached_lens=torch.randint(0, max_len - 8, (B,), generator=g, device=dev).int(),
        slot_ids=torch.randperm(pool, device=dev)[:B].int(),
        num_decoding=torch.tensor([B], dtype=torch.int32, device=dev),
    )
    inv = 1e6 ** (-torch.arange(0, 128, 2, dtype=torch.float32, device=dev) / 128)

    def step():
        ang = static["cached_lens"][:, None, None].float() * inv[None, None, :]
        cos, sin = ang.cos().bfloat16(), ang.sin().bfloat16()
        outs = []
        for li in range(layers):
            x = static["qkv"][li]
            q = x[:, :2048].view(B, 16, 128)
            k = x[:, 2048:3072].view(B, 8, 128)
            v = x[:, 3072:].view(B, 8, 128)
            qo = ie.fused_rope_kv_decode(q, k, v, static["qw"], static["kw"], cos, sin,
                                         static["slot_ids"], caches[li], static["cached_lens"],
                                         static["num_decoding"], 1e-6)
            outs.append(ie.decode_attention(qo, caches[li], static["cached_lens"],
                                            static["slot_ids"], static["num_decoding"],
                                            128 ** -0.5))
        return torch.stack(outs)

    return step, static


def test_decode_graph_replay_bitwise(ie, dev):
    say("graph capture of a 3-layer decode step")
    step, static = _make_step(ie, dev)
    ref = step().clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    junk = torch.randn(512, 512, device=dev)
    for i in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {i} differs from eager"
        junk = junk @ junk.T / 512  # unrelated eager work between replays
        torch.cuda.synchronize()
    # mutate inputs in place: new tokens one position later, new activations
    static["cached_lens"].add_(1)
    static["qkv"].copy_(torch.randn_like(static["qkv"], dtype=torch.float32).bfloat16())
    graph.replay()
    torch.cuda.synchronize()
    eager = step()
    torch.cuda.synchronize()
    assert torch.equal(out, eager), "replay after input mutation differs from eager"
    assert not torch.equal(out, ref)


def test_reference_capture_pattern_shared_pool(ie, workloads, dev):
    """The engine's own capture (engine.py:432-449): warm-up twice on a fresh side stream, then
    torch.cuda.graph(g, pool=pool) on torch's capture stream, where no op has run before. The
    ops' workspaces are then allocated inside each capture from the shared pool, with a recorded
    fill of their arrival counts, so they stay correct when the pool hands the same memory to
    the next graph. Two graphs in one pool (a 3-layer decode step, config 4's prefill attention)
    replay in alternating order, each equal to its eager result every time."""
    step, _ = _make_step(ie, dev)
    wl = workloads.mixed_to(workloads.config4(seed=3), dev)
    gi = wl.inputs

    def prefill():
        return ie.prefill_attention(wl.q, wl.k, wl.v, gi["seq_ids"], gi["cu_seqlens"],
                                    gi["tile_start"], wl.cache, gi["slot_ids"], gi["cu_cached"],
                                    wl.block_m)

    nd = len(wl.decode_ctx)  # prefill attention leaves the decoders' rows of its output unset
    refs = [step().clone(), prefill()[nd:].clone()]
    pool = torch.cuda.graph_pool_handle()
    graphs = []
    for fn in (step, prefill):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                fn()
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, pool=pool):
            out = fn()
        graphs.append((g, out if fn is step else out[nd:]))
    for i, which in enumerate([1, 0, 1, 1, 0, 0, 1]):
        g, out = graphs[which]
        g.replay()
        torch.cuda.synchronize()
        say(f"shared-pool replay {i}: graph {which}")
        assert torch.equal(out, refs[which]), f"replay {i} of graph {which} differs from eager"
