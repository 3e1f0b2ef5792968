"""decode_attention_rope (fused_rope_kv_decode and decode_attention in one launch) on the GPU:
the cache it writes is bit-identical to fused_rope_kv_decode's and to the oracle's, and its
output matches decode_attention on the q that fused_rope_kv_decode returns, and the oracle's
attention on the oracle's q, within the bf16 tolerance."""

import numpy as np
import pytest
import torch

from helpers import assert_attn_close, assert_cache_bitwise, bf16_np, cache_np, cache_to, say
from oracle import attention as oat
from oracle import kv_cache as okv

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5
EPS = 1e-6


def _case(ie, lens, nd, seed, max_len):
    """Raw q/k/v rows of a QKV projection output (strided views), norm weights, RoPE tables at
    the sequences' positions, and a cache whose columns [0, max_len) hold random int8 K/V with
    scales (the new token's column included: the launch must overwrite it)."""
    g = torch.Generator().manual_seed(seed)
    B, hq, hkv = len(lens), 16, 8
    pool = B + 3
    qkv = torch.randn(B, (hq + 2 * hkv) * 128, generator=g).bfloat16()
    q = qkv[:, :hq * 128].view(B, hq, 128)
    k = qkv[:, hq * 128:(hq + hkv) * 128].view(B, hkv, 128)
    v = qkv[:, (hq + hkv) * 128:].view(B, hkv, 128)
    qw = (1 + 0.2 * torch.randn(128, generator=g)).bfloat16()
    kw = (1 + 0.2 * torch.randn(128, generator=g)).bfloat16()
    cached = torch.tensor([n - 1 for n in lens], dtype=torch.int32)
    inv = 1e6 ** (-torch.arange(0, 128, 2, dtype=torch.float32) / 128)
    ang = cached[:, None, None].float() * inv[None, None, :]
    cos, sin = ang.cos().bfloat16(), ang.sin().bfloat16()
    c = ie.make_layer_cache(pool, hkv, max_len, 128, device="cpu")
    c.k.copy_(torch.randint(-127, 128, c.k.shape, generator=g, dtype=torch.int8))
    c.v.copy_(torch.randint(-127, 128, c.v.shape, generator=g, dtype=torch.int8))
    c.k_scale.copy_(torch.rand(c.k_scale.shape, generator=g) * 0.02 + 0.005)
    c.v_scale.copy_(torch.rand(c.v_scale.shape, generator=g) * 0.02 + 0.005)
    c.k_calibration.copy_(torch.rand(c.k_calibration.shape, generator=g) * 3 + 0.01)
    slots = torch.randperm(pool, generator=g)[:B].int()
    return dict(q=q, k=k, v=v, qw=qw, kw=kw, cos=cos, sin=sin, cache=c, slots=slots,
                cached=cached, nd=nd)


@pytest.mark.parametrize("lens,nd", [
    ([1], 1),                                            # the new token is the only one
    ([1, 2, 130, 3000, 7, 257, 64, 65, 900, 4000, 33, 512, 129], 11),  # padding rows after 11
    ([int(x) for x in np.random.default_rng(5).integers(128, 4096, 32)], 32),  # config 5
    ([4096] * 63 + [1], 64),                             # one piece per sequence, full target
    ([int(x) for x in np.random.default_rng(6).integers(1, 600, 300)], 297),  # 2-wave launch
    ([int(x) for x in np.random.default_rng(7).integers(1, 1500, 100)], 100),  # 4-wave launch
])
def test_decode_attention_rope(ie, dev, lens, nd):
    say(f"decode_attention_rope B={len(lens)} nd={nd} max ctx {max(lens)}")
    check_rope(ie, dev, lens, nd)


@pytest.mark.parametrize("seed", range(4))
def test_decode_attention_rope_random(ie, dev, seed):
    """Seeded random batches across the three launch shapes (8-, 4- and 2-wave workgroups):
    1-300 sequences of 1-1,500 tokens, padding rows after num_decoding."""
    rng = np.random.default_rng(200 + seed)
    B = int((rng.integers(1, 65), rng.integers(65, 129), rng.integers(129, 301))[seed % 3])
    lens = [int(x) for x in rng.integers(1, 1501, B)]
    nd = int(rng.integers(max(1, B - 5), B + 1))
    say(f"decode_attention_rope random seed {seed}: B={B} nd={nd} max ctx {max(lens)}")
    check_rope(ie, dev, lens, nd)


def check_rope(ie, dev, lens, nd):
    max_len = -(-max(lens) // 64) * 64
    cs = _case(ie, lens, nd, seed=len(lens), max_len=max_len)
    dv = {n: t.to(dev) for n, t in cs.items() if isinstance(t, torch.Tensor)}
    ndt = torch.tensor([nd], dtype=torch.int32, device=dev)
    # the two reference calls, on one copy of the cache
    c2 = cache_to(cs["cache"], dev, ie.LayerKVCache)
    qo = ie.fused_rope_kv_decode(dv["q"], dv["k"], dv["v"], dv["qw"], dv["kw"], dv["cos"],
                                 dv["sin"], dv["slots"], c2, dv["cached"], ndt, EPS)
    out2 = ie.decode_attention(qo, c2, dv["cached"], dv["slots"], ndt, SCALE)
    # the fused launch, on another
    c1 = cache_to(cs["cache"], dev, ie.LayerKVCache)
    out1 = ie.decode_attention_rope(dv["q"], dv["k"], dv["v"], dv["qw"], dv["kw"], dv["cos"],
                                    dv["sin"], dv["slots"], c1, dv["cached"], ndt, EPS, SCALE)
    torch.cuda.synchronize()
    # the oracle: its fused_rope_kv_decode on a numpy copy, then its decode attention
    ref = cache_np(cs["cache"])
    q_ref = okv.fused_rope_kv_decode(*(bf16_np(cs[n]) for n in ("q", "k", "v", "qw", "kw", "cos",
                                                                "sin")),
                                     cs["slots"].numpy(), ref, cs["cached"].numpy(), nd, EPS)
    assert_cache_bitwise(c1, ref, "decode_attention_rope cache vs oracle")
    assert_cache_bitwise(c1, cache_np(c2), "decode_attention_rope cache vs fused_rope_kv_decode")
    out_ref = oat.decode_attention(q_ref[:nd], ref, cs["cached"].numpy(), cs["slots"].numpy(),
                                   nd, SCALE)
    assert_attn_close(bf16_np(out1)[:nd], out_ref, "fused vs oracle")
    assert_attn_close(bf16_np(out1)[:nd], bf16_np(out2)[:nd], "fused vs two launches")


def test_decode_attention_rope_graph_replays(ie, dev):
    """Captured in a hipGraph and replayed with new positions written in place between
    replays: every replay equals the eager call on the same inputs (output and cache)."""
    say("decode_attention_rope graph replays")
    lens = [int(x) for x in np.random.default_rng(9).integers(100, 2000, 24)]
    cs = _case(ie, lens, len(lens), seed=3, max_len=2304)
    dv = {n: t.to(dev) for n, t in cs.items() if isinstance(t, torch.Tensor)}
    ndt = torch.tensor([len(lens)], dtype=torch.int32, device=dev)
    cg = cache_to(cs["cache"], dev, ie.LayerKVCache)
    out = torch.empty(len(lens), 16, 128, dtype=torch.bfloat16, device=dev)
    run = lambda c, o: ie.decode_attention_rope(dv["q"], dv["k"], dv["v"], dv["qw"], dv["kw"],
                                                dv["cos"], dv["sin"], dv["slots"], c,
                                                dv["cached"], ndt, EPS, SCALE, out=o)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            run(cg, out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        run(cg, out)
    for rep in range(3):
        dv["cached"].add_(rep)  # positions move on; the RoPE tables stay (values only)
        graph.replay()
        torch.cuda.synchronize()
        ce = cache_to(cg, dev, ie.LayerKVCache)
        eager = torch.empty_like(out)
        run(ce, eager)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), f"replay {rep}"
        assert_cache_bitwise(cg, cache_np(ce), f"replay {rep} cache")
