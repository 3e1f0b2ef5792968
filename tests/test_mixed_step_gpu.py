"""A chunked-prefill step through the attention layer's dispatch (qwen3-1.7b/architecture.py:
124-197) as one unit: prefill norm/RoPE -> quantize-on-write -> prefill attention over the
int8 prefix -> decode norm/RoPE/write on q[:B] -> decode attention into the same output.
Checked against the oracle composed the same way: every decode row and every prefill row,
and the whole cache bit for bit afterwards. Then the step as a hipGraph (replay == eager), and
whole-step graphs for several decode batch buckets and token buckets in one memory pool
(engine.py:105-117, 376-449)."""

import importlib

import numpy as np
import pytest
import torch

from helpers import assert_attn_close, assert_cache_bitwise, bf16_np, cache_np, say
from oracle import attention as oat
from oracle import kv_cache as okv

pytestmark = pytest.mark.gpu
HQ, HKV, D = 16, 8, 128
EPS = 1e-6


def _al():
    return importlib.import_module("inference-engine_amd.attention_layer")


def raw_qkv(N, seed, dev):
    """Raw projections of a step (before norm and RoPE): views of one [N, 4096] buffer, as the
    QKV projection's split hands them to the layer."""
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(N, (HQ + 2 * HKV) * D, generator=g).bfloat16().to(dev)
    q = qkv[:, :HQ * D].view(N, HQ, D)
    k = qkv[:, HQ * D:(HQ + HKV) * D].view(N, HKV, D)
    v = qkv[:, (HQ + HKV) * D:].view(N, HKV, D)
    return qkv, q, k, v


def norm_weights(seed, dev):
    g = torch.Generator().manual_seed(seed)
    qw = (1 + 0.2 * torch.randn(D, generator=g)).bfloat16().to(dev)
    kw = (1 + 0.2 * torch.randn(D, generator=g)).bfloat16().to(dev)
    return qw, kw


def oracle_step(q, k, v, qw, kw, cos, sin, cache, ins, block_m):
    """The same step on the oracle: returns (out [N, Hq, D] with NaN in rows the step does not
    write, the cache after the step)."""
    q, k, v, qw, kw, cos, sin = (bf16_np(t) for t in (q, k, v, qw, kw, cos, sin))
    c = cache_np(cache)
    nd = int(ins["num_decoding"][0])
    q_p, k_p = okv.fused_norm_rope_prefill(q, k, qw, kw, cos, sin, EPS)
    okv.quantize_kv_prefill(k_p, v, ins["cu_seqlens"], ins["slot_ids"], ins["cached_lens"], nd, c)
    kp, vp = okv.dequantize_kv_prefix(c, ins["cu_cached"], ins["slot_ids"])
    out = oat.prefill_attention(q_p, k_p, v, ins["cu_seqlens"], ins["tile_start"], block_m, kp,
                                vp, ins["cu_cached"])
    B = len(ins["slot_ids"])
    q_d = okv.fused_rope_kv_decode(q[:B], k[:B], v[:B], qw, kw, cos[:B], sin[:B],
                                   ins["slot_ids"], c, ins["cached_lens"], nd, EPS)
    dec = oat.decode_attention(q_d, c, ins["cached_lens"], ins["slot_ids"], nd, D ** -0.5)
    out[:nd] = dec[:nd]
    return out, c


def run_step(al, wl, q, k, v, qw, kw, cos, sin):
    gi = wl.inputs
    return al.attention(q, k, v, gi["seq_ids"], gi["cu_seqlens"], cos, sin, wl.cache,
                        gi["cached_lens"], gi["slot_ids"], gi["tile_start"], wl.block_m,
                        al.PrefixScratch(None, None, gi["cu_cached"]), gi["num_decoding"], qw,
                        kw, EPS)


def step_setup(workloads, wl, dev, seed):
    al = _al()
    g = workloads.mixed_to(wl, dev)
    N = g.q.shape[0]
    qkv, q, k, v = raw_qkv(N, seed, dev)
    qw, kw = norm_weights(seed + 1, dev)
    inv = al.rope_inv_freq(D, 1e6, dev)
    cos, sin = al.rope_tables(g.inputs["positions"], inv)
    return al, g, qkv, q, k, v, qw, kw, cos, sin


@pytest.mark.parametrize("case", ["config4", "small", "big_entries"])
def test_mixed_step_matches_oracle(ie, workloads, dev, case):
    if case == "config4":
        wl = workloads.config4(seed=4)
    elif case == "small":
        wl = workloads.mixed_workload([9, 300, 1], [(40, 0), (7, 33), (130, 200)], seed=5,
                                      block_m=64, max_len=1024, n_pad=200, num_entries=9)
    else:  # more entries than the prefill kernel stages on chip (engine max_batch_size 960)
        rng = np.random.default_rng(6)
        dctx = [int(x) for x in rng.integers(2, 200, 40)]
        chunks = [(int(rng.integers(1, 4)), int(rng.integers(0, 60))) for _ in range(560)]
        chunks += [(100, 120), (90, 0)]
        wl = workloads.mixed_workload(dctx, chunks, seed=6, block_m=128, max_len=256,
                                      num_entries=961, pool=len(dctx) + len(chunks) + 1)
    nd = int(wl.inputs["num_decoding"][0])
    N = wl.q.shape[0]
    say(f"mixed step {case}: {nd} decoders, {len(wl.chunks)} chunks, N={N}, "
        f"entries={wl.inputs['slot_ids'].shape[0]}")
    al, g, _, q, k, v, qw, kw, cos, sin = step_setup(workloads, wl, dev, seed=7)
    ins = {n: t.cpu().numpy() for n, t in g.inputs.items()}
    ref, ref_cache = oracle_step(q, k, v, qw, kw, cos, sin, g.cache, ins, wl.block_m)
    out = run_step(al, g, q, k, v, qw, kw, cos, sin)
    torch.cuda.synchronize()
    o = bf16_np(out)
    rows = ~np.isnan(ref[:, 0, 0])
    assert rows[:nd].all() and rows[nd:ins["cu_seqlens"][len(wl.decode_ctx) + len(wl.chunks)]].all()
    assert_attn_close(o[:nd], ref[:nd], f"mixed {case}: decode rows")
    assert_attn_close(o[rows], ref[rows], f"mixed {case}: all {int(rows.sum())} rows")
    assert_cache_bitwise(g.cache, ref_cache, f"mixed {case} cache")


def test_mixed_step_graph_replay(ie, workloads, dev):
    """Config 4's step captured as a hipGraph: replays equal the eager step bit for bit, with
    unrelated eager work between them, and after the step's activations change in place."""
    wl = workloads.config4(seed=8)
    al, g, qkv, q, k, v, qw, kw, cos, sin = step_setup(workloads, wl, dev, seed=9)
    run = lambda: run_step(al, g, q, k, v, qw, kw, cos, sin)
    eager = run().clone()
    gs = al.GraphSet()
    graph, out = gs.capture("mixed", run)
    junk = torch.randn(384, 384, device=dev)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i} differs from eager"
        junk = junk @ junk.T / 384
        torch.cuda.synchronize()
    qkv.copy_(torch.randn(qkv.shape, device=dev).bfloat16())
    graph.replay()
    torch.cuda.synchronize()
    got = out.clone()
    want = run()
    torch.cuda.synchronize()
    assert torch.equal(got, want), "replay after input change differs from eager"
    assert not torch.equal(got, eager)


def test_bucket_graphs_share_one_pool(ie, workloads, dev, step_inputs):
    """A two-layer attention stack (AttentionLayer: QKV projection, attention, output
    projection) captured like the engine: decode graphs for batch buckets 1, 2, 4, 8 and
    prefill-step graphs for token buckets 16, 32, 64, all in one pool, each capturing a dummy
    step on the scratch slot; then real steps written into the captured inputs replay equal to
    the eager layers."""
    al = _al()
    ds = importlib.import_module("inference-engine_amd.decode_step")
    torch.manual_seed(0)
    layers_n, pool_slots, max_len, S, block_m = 2, 12, 512, 9, 32
    scratch = pool_slots - 1
    W = ds.random_weights(ds.Qwen3Shape(layers=layers_n, vocab=256), dev, seed=2)[0]
    layers = [al.AttentionLayer(w.qkv, w.o_proj, w.q_norm, w.k_norm) for w in W]
    caches = [ie.make_layer_cache(pool_slots, HKV, max_len, D, device=dev) for _ in W]
    gen = torch.Generator(device=dev).manual_seed(3)
    for c in caches:
        c.k.copy_(torch.randint(-127, 128, c.k.shape, generator=gen, device=dev, dtype=torch.int8))
        c.v.copy_(torch.randint(-127, 128, c.v.shape, generator=gen, device=dev, dtype=torch.int8))
        c.k_scale.copy_(torch.rand(c.k_scale.shape, generator=gen, device=dev) * 0.05)
        c.v_scale.copy_(torch.rand(c.v_scale.shape, generator=gen, device=dev) * 0.05)
    inv = al.rope_inv_freq(D, 1e6, dev)
    x_all = torch.randn(64, 2048, device=dev).bfloat16()
    gs = al.GraphSet()

    # decode: fixed tensors sliced per bucket (engine.py:376-406)
    Bmax = 8
    d_cl = torch.zeros(Bmax, dtype=torch.int32, device=dev)
    d_slot = torch.full((Bmax,), scratch, dtype=torch.int32, device=dev)
    d_x = torch.zeros(Bmax, 2048, dtype=torch.bfloat16, device=dev)
    nds = {}

    def decode_run(b):
        def run():
            cos, sin = al.rope_tables(d_cl[:b], inv)
            h = d_x[:b]
            for li, lay in enumerate(layers):
                h = lay(h, None, None, cos, sin, caches[li], d_cl[:b], d_slot[:b], None, block_m,
                        None, nds[b])
            return h
        return run

    for b in (8, 4, 2, 1):
        nds[b] = torch.full((1,), b, dtype=torch.int32, device=dev)
        gs.capture(("decode", b), decode_run(b))

    # prefill steps: one input buffer, per-bucket views (engine.py:414-430)
    buckets = [16, 32, 64]
    lay_max = sum(step_inputs.input_layout(64, S, block_m))
    buf = torch.zeros(lay_max, dtype=torch.int32, device=dev)
    p_x = torch.zeros(64, 2048, dtype=torch.bfloat16, device=dev)
    names = ["ids", "positions", "seq_ids", "cu_seqlens", "cached_lens", "slot_ids", "cu_cached",
             "tile_start", "num_decoding"]

    def views(n):
        lay = step_inputs.input_layout(n, S, block_m)
        return dict(zip(names, buf[:sum(lay)].split(lay)))

    def write(st):
        flat = torch.tensor([x for f in st.fields() for x in f], dtype=torch.int32)
        buf[:len(flat)].copy_(flat)

    def prefill_run(n):
        v_ = views(n)

        def run():
            cos, sin = al.rope_tables(v_["positions"], inv)
            h = p_x[:n]
            for li, lay in enumerate(layers):
                h = lay(h, v_["seq_ids"], v_["cu_seqlens"], cos, sin, caches[li],
                        v_["cached_lens"], v_["slot_ids"], v_["tile_start"], block_m,
                        al.PrefixScratch(None, None, v_["cu_cached"]), v_["num_decoding"])
            return h
        return run

    for n in reversed(buckets):
        write(step_inputs.fill_inputs([], 0, n, S, block_m, scratch))  # dummy: padding only
        gs.capture(("prefill", n), prefill_run(n))

    # real steps replayed through the captured graphs, each against the same layers run eagerly
    for b, lens in ((3, [40, 200, 7]), (8, [1, 2, 3, 4, 300, 301, 9, 77]), (1, [130])):
        bb = next(x for x in (1, 2, 4, 8) if x >= b)
        d_cl.fill_(0)
        d_slot.fill_(scratch)
        d_cl[:b] = torch.tensor(lens, dtype=torch.int32)
        d_slot[:b] = torch.arange(b, dtype=torch.int32)
        d_x[:bb] = x_all[:bb]
        want = decode_run(bb)().clone()
        got = gs.replay(("decode", bb))
        torch.cuda.synchronize()
        say(f"decode bucket {bb} (B={b}) replay == eager")
        assert torch.equal(got, want)
    plans = [
        (2, [(40, 0, [5]), (100, 1, [6]), (0, 2, [1] * 9)], 16),
        (1, [(70, 3, [5]), (20, 4, [1] * 20)], 32),
        (3, [(10, 5, [1]), (11, 6, [2]), (12, 7, [3]), (33, 8, [4] * 30), (0, 9, [4] * 12)], 64),
    ]
    for nd, plan, n in plans:
        write(step_inputs.fill_inputs(plan, nd, n, S, block_m, scratch))
        p_x[:n] = x_all[:n]
        want = prefill_run(n)().clone()
        got = gs.replay(("prefill", n))
        torch.cuda.synchronize()
        say(f"prefill bucket {n} ({nd} decoding, {len(plan) - nd} prefilling) replay == eager")
        assert torch.equal(got, want)
