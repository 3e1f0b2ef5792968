"""Other attention geometries than Qwen3-1.7B's 16 query / 8 KV heads: GQA ratios 1, 4, 5, 8 and
16 (the other Qwen3 sizes: 32/8 for 4B and 8B, 40/8 for 14B, 64/8 for 32B, 64/4 for the 235B
MoE) and the one-GPU share of an 8-way tensor-parallel layer (2 query heads over 1 KV head),
through decode attention (plain and fused with the KV write), prefill attention and a whole
mixed step of the attention layer, against the oracle (which takes any ratio: query head h
reads KV head h // ratio, kernels.py:118-135). head_dim stays 128, the only one the kernels take.
"""

import importlib

import numpy as np
import pytest
import torch

from helpers import assert_attn_close, assert_cache_bitwise, bf16_np, cache_np, say
from oracle import attention as oat
from oracle import kv_cache as okv

pytestmark = pytest.mark.gpu
D = 128
SCALE = D ** -0.5
GEOMETRIES = [(8, 8), (32, 8), (40, 8), (64, 8), (64, 4), (2, 1)]


def _decode_ref(wl):
    c = cache_np(wl.cache)
    return oat.decode_attention(bf16_np(wl.q), c, wl.cached_lens.numpy(), wl.slot_ids.numpy(),
                                int(wl.num_decoding[0]), SCALE)


@pytest.mark.parametrize("hq,hkv", GEOMETRIES)
def test_decode_geometry(ie, workloads, dev, hq, hkv):
    """Ragged sequences (one token to 4,096: single pieces and split ones merged in the launch),
    and a partial batch: rows past num_decoding untouched."""
    ctx = [300, 2000, 77, 4096, 1, 1500]
    say(f"decode hq={hq} hkv={hkv} ctx {ctx}")
    wl = workloads.decode_workload(ctx, seed=21, hq=hq, hkv=hkv, num_decoding=5)
    ref = _decode_ref(wl)
    g = wl.to(dev)
    out = torch.full_like(g.q, 7.0)
    ie.decode_attention(g.q, g.cache, g.cached_lens, g.slot_ids, g.num_decoding, SCALE, out=out)
    torch.cuda.synchronize()
    o = bf16_np(out)
    assert_attn_close(o[:5], ref[:5], f"decode {hq}/{hkv}")
    assert (o[5:] == 7.0).all(), "row past num_decoding written"


@pytest.mark.parametrize("hq,hkv", [(2, 1), (32, 8)])
def test_decode_headline_shapes(ie, workloads, dev, hq, hkv):
    """B=64, ctx=4096 at the tensor-parallel share (2 query heads over 1 KV head: one GPU's part
    of an 8-way split of the 16/8 layer) and at GQA 4 (32/8)."""
    say(f"decode B=64 ctx=4096 hq={hq} hkv={hkv}")
    wl = workloads.decode_workload([4096] * 64, seed=22, hq=hq, hkv=hkv)
    ref = _decode_ref(wl)
    g = wl.to(dev)
    out = ie.decode_attention(g.q, g.cache, g.cached_lens, g.slot_ids, g.num_decoding, SCALE)
    torch.cuda.synchronize()
    assert_attn_close(bf16_np(out), ref, f"decode headline {hq}/{hkv}")


@pytest.mark.parametrize("hq,hkv", [(32, 8), (40, 8), (8, 8), (2, 1)])
def test_decode_rope_geometry(ie, dev, hq, hkv):
    """The fused decode launch (norm, RoPE and the new token's K/V write, then attention): the
    cache bit for bit as fused_rope_kv_decode writes it (one writer per KV head, whatever the
    number of query-head pairs) and the outputs against the oracle."""
    say(f"decode_attention_rope hq={hq} hkv={hkv}")
    g = torch.Generator().manual_seed(23)
    B, pool, L = 9, 12, 2304
    qkv = torch.randn(B, (hq + 2 * hkv) * D, generator=g).bfloat16()
    q = qkv[:, :hq * D].view(B, hq, D)
    k = qkv[:, hq * D:(hq + hkv) * D].view(B, hkv, D)
    v = qkv[:, (hq + hkv) * D:].view(B, hkv, D)
    qw = (1 + 0.2 * torch.randn(D, generator=g)).bfloat16()
    kw = (1 + 0.2 * torch.randn(D, generator=g)).bfloat16()
    lens = torch.tensor([0, 5, 130, 700, 2000, 2200, 64, 1023, 333], dtype=torch.int32)
    slots = torch.randperm(pool, generator=g)[:B].int()
    inv = 1e6 ** (-torch.arange(0, D, 2, dtype=torch.float32) / D)
    ang = lens[:, None, None].float() * inv[None, None, :]
    cos, sin = ang.cos().bfloat16(), ang.sin().bfloat16()
    c = ie.make_layer_cache(pool, hkv, L, D, device="cpu")
    c.k.copy_(torch.randint(-127, 128, c.k.shape, generator=g, dtype=torch.int8))
    c.v.copy_(torch.randint(-127, 128, c.v.shape, generator=g, dtype=torch.int8))
    c.k_scale.copy_(torch.rand(c.k_scale.shape, generator=g) * 0.05)
    c.v_scale.copy_(torch.rand(c.v_scale.shape, generator=g) * 0.05)
    c.k_calibration.copy_(torch.rand(c.k_calibration.shape, generator=g) * 2 + 0.1)
    nd = 8
    ref_c = cache_np(c)
    q_d = okv.fused_rope_kv_decode(*(bf16_np(t) for t in (q, k, v, qw, kw, cos, sin)),
                                   slots.numpy(), ref_c, lens.numpy(), nd, 1e-6)
    ref = oat.decode_attention(q_d, ref_c, lens.numpy(), slots.numpy(), nd, SCALE)
    gc = ie.LayerKVCache(*(t.to(dev) for t in (c.k, c.v, c.k_scale, c.v_scale, c.k_calibration)))
    out = torch.zeros(B, hq, D, dtype=torch.bfloat16, device=dev)
    ie.decode_attention_rope(*(t.to(dev) for t in (q, k, v, qw, kw, cos, sin, slots)), gc,
                             lens.to(dev), torch.tensor([nd], dtype=torch.int32, device=dev),
                             1e-6, SCALE, out=out)
    torch.cuda.synchronize()
    assert_cache_bitwise(gc, ref_c, f"decode_attention_rope {hq}/{hkv} cache")
    # V here reaches 127 * 0.05: outputs of magnitude up to ~4, where one bf16 step is 2^-6
    assert_attn_close(bf16_np(out)[:nd], ref[:nd], f"decode_attention_rope {hq}/{hkv}",
                      abs_scale=max(1.0, float(np.abs(ref[:nd]).max())))


@pytest.mark.parametrize("hq,hkv", [(32, 8), (40, 8), (8, 8), (64, 4), (2, 1)])
def test_prefill_geometry(ie, workloads, dev, hq, hkv):
    """Chunks with and without a cached prefix, long enough for split pieces merged in the
    launch: every prefill row against the oracle."""
    chunks = [(200, 300), (64, 0), (129, 1000)]
    say(f"prefill hq={hq} hkv={hkv} chunks {chunks}")
    wl = workloads.mixed_workload([7, 40], chunks, seed=24, block_m=128, max_len=1216, hq=hq,
                                  hkv=hkv)
    ins = {n: t.numpy() for n, t in wl.inputs.items()}
    kp, vp = okv.dequantize_kv_prefix(cache_np(wl.cache), ins["cu_cached"], ins["slot_ids"])
    ref = oat.prefill_attention(bf16_np(wl.q), bf16_np(wl.k), bf16_np(wl.v), ins["cu_seqlens"],
                                ins["tile_start"], wl.block_m, kp, vp, ins["cu_cached"])
    g = workloads.mixed_to(wl, dev)
    gi = g.inputs
    out = ie.prefill_attention(g.q, g.k, g.v, gi["seq_ids"], gi["cu_seqlens"], gi["tile_start"],
                               g.cache, gi["slot_ids"], gi["cu_cached"], g.block_m)
    torch.cuda.synchronize()
    cov = ~np.isnan(ref[:, 0, 0])
    assert cov.sum() == sum(L for L, _ in chunks)
    assert_attn_close(bf16_np(out)[cov], ref[cov], f"prefill {hq}/{hkv}")


@pytest.mark.parametrize("hq,hkv", [(32, 8), (40, 8)])
def test_mixed_step_geometry(ie, workloads, dev, hq, hkv):
    """A config-4-shaped step (30 decoders, a 512-token first chunk, 512 tokens after 1,536
    cached) through the attention layer at 32/8 and 40/8 heads: prefill norm/RoPE, KV write,
    prefill attention and the fused decode, every row against the oracle and the cache bit for
    bit afterwards."""
    ms = importlib.import_module("test_mixed_step_gpu")
    al = importlib.import_module("inference-engine_amd.attention_layer")
    g0 = torch.Generator().manual_seed(25)
    dctx = torch.randint(128, 2049, (30,), generator=g0).tolist()
    wl = workloads.mixed_workload(dctx, [(512, 0), (512, 1536)], seed=25, hq=hq, hkv=hkv)
    say(f"mixed step hq={hq} hkv={hkv}: N={wl.q.shape[0]}")
    g = workloads.mixed_to(wl, dev)
    N = g.q.shape[0]
    qkv = torch.randn(N, (hq + 2 * hkv) * D, generator=g0).bfloat16().to(dev)
    q = qkv[:, :hq * D].view(N, hq, D)
    k = qkv[:, hq * D:(hq + hkv) * D].view(N, hkv, D)
    v = qkv[:, (hq + hkv) * D:].view(N, hkv, D)
    qw, kw = ms.norm_weights(26, dev)
    cos, sin = al.rope_tables(g.inputs["positions"], al.rope_inv_freq(D, 1e6, dev))
    ins = {n: t.cpu().numpy() for n, t in g.inputs.items()}
    ref, ref_cache = ms.oracle_step(q, k, v, qw, kw, cos, sin, g.cache, ins, wl.block_m)
    out = ms.run_step(al, g, q, k, v, qw, kw, cos, sin)
    torch.cuda.synchronize()
    o = bf16_np(out)
    rows = ~np.isnan(ref[:, 0, 0])
    assert_attn_close(o[:30], ref[:30], f"mixed {hq}/{hkv}: decode rows")
    assert_attn_close(o[rows], ref[rows], f"mixed {hq}/{hkv}: all rows")
    assert_cache_bitwise(g.cache, ref_cache, f"mixed {hq}/{hkv} cache")


def test_workspace_shared_across_head_counts(ie, workloads, dev):
    """Decode calls of different head counts on one stream share the op's kept workspace: a
    2/1 call (two query heads: few count words, partials right after them) followed by a 16/8
    call of 300 sequences, whose count words for sequences 256 and up lie where the 2/1 call's
    partials would have been had the count region been sized by the call's own head count.
    Every row of the second call against the oracle."""
    small = workloads.decode_workload([3000, 700, 4096, 20], seed=26, hq=2, hkv=1).to(dev)
    ie.decode_attention(small.q, small.cache, small.cached_lens, small.slot_ids,
                        small.num_decoding, SCALE)
    ctx = [int(x) for x in np.random.default_rng(27).integers(1, 601, 300)]
    wl = workloads.decode_workload(ctx, seed=27, num_decoding=299)
    ref = _decode_ref(wl)
    g = wl.to(dev)
    for rep in range(2):
        out = ie.decode_attention(g.q, g.cache, g.cached_lens, g.slot_ids, g.num_decoding, SCALE)
        torch.cuda.synchronize()
        assert_attn_close(bf16_np(out)[:299], ref[:299], f"16/8 after 2/1, call {rep}")
        ie.decode_attention(small.q, small.cache, small.cached_lens, small.slot_ids,
                            small.num_decoding, SCALE)
