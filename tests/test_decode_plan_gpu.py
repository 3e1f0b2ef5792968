"""decode_attention / decode_attention_rope with the step's work list computed once (decode_plan,
then ie_decode_attention_planned / ie_decode_attention_rope_planned): outputs and cache writes
bit for bit equal to the launches that derive the list from cached_lens themselves, over the
launch shapes (8-, 4- and 2-wave workgroups, one piece per sequence, split sequences, padding
rows past num_decoding), other GQA ratios, one plan serving two layers, and a replayed graph
whose inputs change between replays. The self-scheduling launches are the ones the oracle tests
pin (test_decode_gpu.py, test_decode_rope_gpu.py); one case here is also checked against the
oracle directly."""

import numpy as np
import pytest
import torch

from helpers import assert_attn_close, bf16_np, cache_np, cache_to, say
from oracle import attention as oat
from test_decode_rope_gpu import _case

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5
EPS = 1e-6
SHAPES = [
    ([int(x) for x in np.random.default_rng(5).integers(128, 4096, 32)], 32),  # config 5
    ([4096] * 63 + [1], 64),                    # one piece per sequence
    ([1, 2, 130, 3000, 7, 257, 64, 65, 900, 4000, 33, 512, 129], 11),  # padding rows
    ([int(x) for x in np.random.default_rng(7).integers(1, 1500, 100)], 100),  # 4 waves
    ([int(x) for x in np.random.default_rng(6).integers(1, 600, 300)], 297),   # 2 waves
]


def _fields(c):
    return (c.k, c.v, c.k_scale, c.v_scale, c.k_calibration)


def _gpu(ie, c, dev):
    g = {n: (t.to(dev) if torch.is_tensor(t) else t) for n, t in c.items() if n != "cache"}
    g["cache"] = cache_to(c["cache"], dev, ie.LayerKVCache)
    g["nd_t"] = torch.tensor([c["nd"]], dtype=torch.int32, device=dev)
    return g


def _plan(ie, g, hq=16, hkv=8):
    return ie.decode_plan(g["cached"], g["nd_t"], g["q"].shape[0], hq, hkv)


def _rope(ie, g, cache, plan=None):
    out = torch.full_like(g["q"], 3.0)
    ie.decode_attention_rope(g["q"], g["k"], g["v"], g["qw"], g["kw"], g["cos"], g["sin"],
                             g["slots"], cache, g["cached"], g["nd_t"], EPS, SCALE, out=out,
                             plan=plan)
    return out


@pytest.mark.parametrize("lens,nd", SHAPES)
def test_planned_decode_rope_equals_self_scheduled(ie, dev, lens, nd):
    say(f"planned decode_attention_rope B={len(lens)} nd={nd}")
    g = _gpu(ie, _case(ie, lens, nd, 50 + len(lens), max(lens) + 8), dev)
    c2 = cache_to(g["cache"], dev, ie.LayerKVCache)
    plan = _plan(ie, g)
    base = _rope(ie, g, g["cache"])
    planned = _rope(ie, g, c2, plan)
    torch.cuda.synchronize()
    assert torch.equal(base, planned), "planned launch output differs"
    for a, b in zip(_fields(g["cache"]), _fields(c2)):
        assert torch.equal(a, b), "planned launch cache differs"


@pytest.mark.parametrize("lens,nd", SHAPES[:3])
def test_planned_decode_equals_self_scheduled(ie, dev, lens, nd):
    say(f"planned decode_attention B={len(lens)} nd={nd}")
    g = _gpu(ie, _case(ie, lens, nd, 60 + len(lens), max(lens) + 8), dev)
    q = g["q"].contiguous()
    plan = _plan(ie, g)
    outs = []
    for p in (None, plan):
        o = torch.full_like(q, 3.0)
        ie.decode_attention(q, g["cache"], g["cached"], g["slots"], g["nd_t"], SCALE, out=o,
                            plan=p)
        outs.append(o)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    if len(lens) == 32:  # config 5 against the oracle directly
        c = cache_np(g["cache"])
        ref = oat.decode_attention(bf16_np(q), c, g["cached"].cpu().numpy(),
                                   g["slots"].cpu().numpy(), nd, SCALE)
        assert_attn_close(bf16_np(outs[1])[:nd], ref[:nd], "planned decode, config 5")


@pytest.mark.parametrize("hq,hkv", [(40, 8), (2, 1), (8, 8)])
def test_planned_decode_other_ratios(ie, workloads, dev, hq, hkv):
    ctx = [300, 2000, 77, 4096, 1, 1500]
    wl = workloads.decode_workload(ctx, seed=61, hq=hq, hkv=hkv, num_decoding=5).to(dev)
    plan = ie.decode_plan(wl.cached_lens, wl.num_decoding, len(ctx), hq, hkv)
    outs = []
    for p in (None, plan):
        o = torch.full_like(wl.q, 7.0)
        ie.decode_attention(wl.q, wl.cache, wl.cached_lens, wl.slot_ids, wl.num_decoding, SCALE,
                            out=o, plan=p)
        outs.append(o)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]), f"{hq}/{hkv}"


def test_one_plan_two_layers_in_graph(ie, dev):
    """A graph computing the plan once and running two layers' fused decode launches from it,
    replayed three times with new lengths (every sequence one token longer) and new q rows in
    between: every replay equals the eager self-scheduled launches on the same inputs."""
    lens = [int(x) for x in np.random.default_rng(8).integers(128, 2048, 24)]
    c = _case(ie, lens, 24, 70, max(lens) + 16)
    g = _gpu(ie, c, dev)
    caches = [g["cache"], cache_to(g["cache"], dev, ie.LayerKVCache)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())

    def step():
        plan = _plan(ie, g)
        return [_rope(ie, g, cc, plan) for cc in caches]

    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        outs = step()
    gen = torch.Generator().manual_seed(71)
    for rep in range(3):
        g["cached"].add_(1)
        g["q"].copy_(torch.randn(g["q"].shape, generator=gen).bfloat16())
        ref_caches = [cache_to(cc, dev, ie.LayerKVCache) for cc in caches]
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        refs = [_rope(ie, g, cc) for cc in ref_caches]
        torch.cuda.synchronize()
        for i in range(2):
            assert torch.equal(outs[i], refs[i]), f"replay {rep} layer {i}"
            for a, b in zip(_fields(caches[i]), _fields(ref_caches[i])):
                assert torch.equal(a, b), f"replay {rep} layer {i} cache"


def test_step_prologue_equals_separate_calls(ie, dev):
    """decode_step_prologue (one launch) against the three calls it replaces on the same inputs:
    the embedding rows, decode_plan's work list and rope_tables' cos / sin, bit for bit; an id
    outside the vocabulary gives a zero row."""
    import torch.nn.functional as F
    g = torch.Generator().manual_seed(81)
    V, D, B = 1000, 256, 32
    embed = torch.randn(V, D, generator=g).bfloat16().to(dev)
    ids = torch.randint(0, V, (B, 1), generator=g).to(dev)
    lens = torch.randint(1, 4096, (B,), generator=g).int().to(dev)
    nd = torch.tensor([B - 3], dtype=torch.int32, device=dev)
    inv = ie.attention_layer.rope_inv_freq(128, 1e6, dev)
    x, plan, cos, sin = ie.decode_step_prologue(ids, embed, lens, nd, 16, 8, inv)
    x0 = F.embedding(ids.view(-1), embed)
    plan0 = ie.decode_plan(lens, nd, B, 16, 8)
    cos0, sin0 = ie.attention_layer.rope_tables(lens, inv)
    torch.cuda.synchronize()
    assert torch.equal(x, x0) and torch.equal(plan, plan0)
    assert torch.equal(cos, cos0) and torch.equal(sin, sin0)
    bad = ids.clone()
    bad[5, 0] = V + 7
    xb = ie.decode_step_prologue(bad, embed, lens, nd, 16, 8, inv)[0]
    torch.cuda.synchronize()
    assert torch.all(xb[5] == 0) and torch.equal(xb[:5], x0[:5])
