"""int8 quantize-on-write and prefix dequantize on the GPU: bit-exact against the oracle."""

import numpy as np
import pytest
import torch

from helpers import assert_cache_bitwise, bf16_np, cache_np, cache_to, say
from oracle import kv_cache as okv
from oracle.numerics import bf16_bits

pytestmark = pytest.mark.gpu


def _prefill_case(workloads, decode_ctx, chunks, seed, max_len=2048):
    wl = workloads.mixed_workload(decode_ctx, chunks, seed=seed, block_m=128, max_len=max_len)
    return wl


@pytest.mark.parametrize("decode_ctx,chunks", [
    ("config4", None),
    ([3, 70], [(1, 0), (17, 0), (0, 0), (33, 5), (1000, 0)]),
    ([], [(2100, 0), (129, 300)]),
    ([5, 9], [(4000, 0), (64, 0), (1, 0), (300, 700)]),
])
def test_quantize_kv_prefill_bitwise(ie, workloads, dev, decode_ctx, chunks):
    # steps of more than 1536 packed tokens compute a first chunk's calibration in two launches
    # ahead of the quantize launch (the last two cases), shorter ones inside it
    say(f"quantize_kv_prefill case {decode_ctx if chunks is None else chunks}")
    if decode_ctx == "config4":
        wl = workloads.config4(seed=3)
    else:
        wl = _prefill_case(workloads, decode_ctx, chunks, seed=4, max_len=4096)
    ins = {n: t.numpy() for n, t in wl.inputs.items()}
    ref = cache_np(wl.cache)
    okv.quantize_kv_prefill(bf16_np(wl.k), bf16_np(wl.v), ins["cu_seqlens"], ins["slot_ids"],
                            ins["cached_lens"], int(ins["num_decoding"][0]), ref)
    g = workloads.mixed_to(wl, dev)
    gi = g.inputs
    assert g.v.stride(0) == 32 * 128  # strided view of a fused qkv row
    ie.quantize_kv_prefill(g.k, g.v, gi["cu_seqlens"], gi["slot_ids"], gi["cached_lens"],
                           gi["num_decoding"], g.cache)
    torch.cuda.synchronize()
    assert_cache_bitwise(g.cache, ref, "quantize_kv_prefill")


def test_fused_rope_kv_decode_bitwise(ie, dev):
    say("fused_rope_kv_decode bitwise")
    g = torch.Generator().manual_seed(5)
    B, hq, hkv, pool, L = 13, 16, 8, 17, 96
    qkv = torch.randn(B, (hq + 2 * hkv) * 128, generator=g).bfloat16()
    q = qkv[:, :hq * 128].view(B, hq, 128)
    k = qkv[:, hq * 128:(hq + hkv) * 128].view(B, hkv, 128)
    v = qkv[:, (hq + hkv) * 128:].view(B, hkv, 128)
    qw = (1 + 0.2 * torch.randn(128, generator=g)).bfloat16()
    kw = (1 + 0.2 * torch.randn(128, generator=g)).bfloat16()
    pos = torch.randint(0, 4000, (B,), generator=g)
    inv = 1e6 ** (-torch.arange(0, 128, 2, dtype=torch.float32) / 128)
    ang = pos[:, None, None].float() * inv[None, None, :]
    cos, sin = ang.cos().bfloat16(), ang.sin().bfloat16()
    c = ie.make_layer_cache(pool, hkv, L, 128, device="cpu")
    c.k_calibration.copy_(torch.rand(c.k_calibration.shape, generator=g) * 3 + 0.01)
    slots = torch.randperm(pool, generator=g)[:B].int()
    lens = torch.randint(0, L, (B,), generator=g).int()
    nd = 11
    ref = cache_np(c)
    qo_ref = okv.fused_rope_kv_decode(*(bf16_np(t) for t in (q, k, v, qw, kw, cos, sin)),
                                      slots.numpy(), ref, lens.numpy(), nd, 1e-6)
    gc = cache_to(c, dev, ie.LayerKVCache)
    qo = ie.fused_rope_kv_decode(*(t.to(dev) for t in (q, k, v, qw, kw, cos, sin, slots)), gc,
                                 lens.to(dev), torch.tensor([nd], dtype=torch.int32, device=dev),
                                 1e-6)
    torch.cuda.synchronize()
    assert_cache_bitwise(gc, ref, "fused_rope_kv_decode")
    got = qo.cpu().view(torch.int16).numpy().view(np.uint16)[:nd]
    exp = bf16_bits(qo_ref[:nd])
    assert np.array_equal(got, exp), f"q_out mismatches: {np.count_nonzero(got != exp)}"


def test_dequantize_kv_prefix_bitwise(ie, workloads, dev):
    say("dequantize_kv_prefix bitwise")
    wl = workloads.mixed_workload([50, 7], [(20, 300), (5, 0), (9, 1031)], seed=8, max_len=2048)
    ins = {n: t.numpy() for n, t in wl.inputs.items()}
    ref_k, ref_v = okv.dequantize_kv_prefix(cache_np(wl.cache), ins["cu_cached"], ins["slot_ids"])
    g = workloads.mixed_to(wl, dev)
    total = int(ins["cu_cached"][-1])
    ko = torch.zeros(8, total + 5, 128, dtype=torch.bfloat16, device=dev)
    vo = torch.zeros_like(ko)
    ie.dequantize_kv_prefix(g.cache, g.inputs["cu_cached"], g.inputs["slot_ids"], ko, vo)
    torch.cuda.synchronize()
    kb = ko.cpu().view(torch.int16).numpy().view(np.uint16)
    vb = vo.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(kb[:, :total], bf16_bits(ref_k))
    assert np.array_equal(vb[:, :total], bf16_bits(ref_v))
    assert not kb[:, total:].any()


@pytest.mark.parametrize("long_step", [False, True])
def test_quantize_kv_prefill_edge_values_bitwise(ie, workloads, dev, long_step):
    """Rows the reciprocal division does not serve (a K or V value of magnitude 2^100 or more:
    those rows take the IEEE division), rows of subnormal and of zero values, V rows whose
    quotients are exact halves (round half to even), and a continuing chunk whose calibration
    row holds arbitrary fp32 values: bit-exact against the oracle, in the one-launch form and in
    the long form (calibration launches, then the streaming quantize launch)."""
    chunks = [(2000, 0), (300, 150)] if long_step else [(300, 0), (200, 150)]
    say(f"quantize_kv_prefill edge values, chunks {chunks}")
    wl = _prefill_case(workloads, [4], chunks, seed=9, max_len=4096)
    rng = np.random.default_rng(9)
    k, v = wl.k.float(), wl.v.float()
    cu = wl.inputs["cu_seqlens"].numpy()
    r = lambda e: int(cu[e]) + int(rng.integers(0, chunks[e - 1][0]))
    k[r(1), 3] *= 2.0 ** 105            # first chunk: raises that channel's calibration too
    k[r(2), 5, 17] = 2.0 ** 101          # continuing chunk: one huge value in a row
    v[r(1), 2, 7] = -(2.0 ** 110)
    k[r(1), 6] = torch.from_numpy(rng.choice([-1, 1], 128) * 2.0 ** -130).float()  # subnormal
    v[r(2), 1] = 0.0
    halves = torch.from_numpy(np.concatenate([[127.0], np.arange(127) - 63.5])).float()
    v[r(1), 4] = halves                  # scale 1: quotients -63.5 ... 62.5
    v[r(2), 0] = -halves
    wl.k.copy_(k.bfloat16())
    wl.v.copy_(v.bfloat16())
    slot_cont = int(wl.inputs["slot_ids"][2])
    wl.cache.k_calibration[slot_cont] = torch.from_numpy(
        np.exp(rng.uniform(np.log(1e-3), np.log(50.0), (8, 1, 128)))).float()
    ins = {n: t.numpy() for n, t in wl.inputs.items()}
    ref = cache_np(wl.cache)
    okv.quantize_kv_prefill(bf16_np(wl.k), bf16_np(wl.v), ins["cu_seqlens"], ins["slot_ids"],
                            ins["cached_lens"], int(ins["num_decoding"][0]), ref)
    g = workloads.mixed_to(wl, dev)
    gi = g.inputs
    ie.quantize_kv_prefill(g.k, g.v, gi["cu_seqlens"], gi["slot_ids"], gi["cached_lens"],
                           gi["num_decoding"], g.cache)
    torch.cuda.synchronize()
    assert_cache_bitwise(g.cache, ref, "quantize_kv_prefill edge values")
