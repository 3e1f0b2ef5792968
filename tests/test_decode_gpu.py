"""Split-K decode attention on the GPU against the oracle (bf16 tolerance), through the torch
op and through the C ABI, at BASELINE configs 1-3 and ragged edge cases."""

import ctypes

import numpy as np
import pytest
import torch

from helpers import assert_attn_close, bf16_np, cache_np, say
from oracle import attention as oat

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5


def oracle_out(wl, nd=None, rows=None):
    nd = len(wl.ctx) if nd is None else nd
    return oat.decode_attention(bf16_np(wl.q), cache_np(wl.cache), wl.cached_lens.cpu().numpy(),
                                wl.slot_ids.cpu().numpy(), nd, SCALE)


@pytest.mark.parametrize("cfg", ["1", "2", "3:16:1024", "3:64:1024"])
def test_decode_configs(ie, workloads, dev, cfg):
    ctx = workloads.decode_ctx_lens(cfg)
    say(f"decode config {cfg}: B={len(ctx)} ctx {min(ctx)}..{max(ctx)}")
    wl = workloads.decode_workload(ctx, seed=21)
    ref = oracle_out(wl)
    g = wl.to(dev)
    out = ie.decode_attention(g.q, g.cache, g.cached_lens, g.slot_ids, g.num_decoding, SCALE)
    torch.cuda.synchronize()
    assert_attn_close(bf16_np(out), ref, f"decode {cfg}")


@pytest.mark.parametrize("ctx", [
    [1], [2, 1, 3], [5, 127, 128, 129, 255, 256, 257], [33000], [64] * 40 + [9000],
    list(range(1, 300, 7)),
    # batches at and just under the per-head workgroup target (64 on 256 CUs), where the grid
    # has no spare workgroups and the fitted piece must keep every piece inside it
    [int(x) for x in np.random.default_rng(7).integers(1, 3000, 64)],
    [int(x) for x in np.random.default_rng(8).integers(100, 5000, 63)],
    [4096] * 63 + [1],
])
def test_decode_ragged(ie, workloads, dev, ctx):
    say(f"decode ragged B={len(ctx)} max ctx {max(ctx)}")
    wl = workloads.decode_workload(ctx, seed=len(ctx), pool=len(ctx) + 3)
    ref = oracle_out(wl)
    g = wl.to(dev)
    out = ie.decode_attention(g.q, g.cache, g.cached_lens, g.slot_ids, g.num_decoding, SCALE)
    torch.cuda.synchronize()
    assert_attn_close(bf16_np(out), ref, f"ragged {len(ctx)}")


def test_decode_partial_batch_and_out_rows(ie, workloads, dev):
    """Rows >= num_decoding of `out` are untouched; out may be taller than B (mixed steps)."""
    ctx = [700, 40, 1500, 3, 64, 900]
    wl = workloads.decode_workload(ctx, seed=9, num_decoding=4)
    ref = oracle_out(wl, nd=4)
    g = wl.to(dev)
    out = torch.full((len(ctx) + 10, 16, 128), 7.0, dtype=torch.bfloat16, device=dev)
    ie.decode_attention(g.q, g.cache, g.cached_lens, g.slot_ids, g.num_decoding, SCALE, out=out)
    torch.cuda.synchronize()
    o = bf16_np(out)
    assert_attn_close(o[:4], ref[:4], "partial batch")
    assert np.all(o[4:] == 7.0)


def test_decode_full_size_sampled(ie, workloads, dev):
    """B=64, ctx=4096 (the headline shape), generated on the GPU; 6 sampled sequences checked
    against the oracle on their own rows, all outputs finite and bounded by max|v|."""
    ctx = [4096] * 64
    say("decode headline shape B=64 ctx=4096 (sampled)")
    g = workloads.decode_workload(ctx, seed=1, device=dev)
    out = ie.decode_attention(g.q, g.cache, g.cached_lens, g.slot_ids, g.num_decoding, SCALE)
    torch.cuda.synchronize()
    o = bf16_np(out)
    assert np.isfinite(o).all()
    pick = [0, 5, 17, 32, 50, 63]
    sub = workloads.DecodeWorkload(
        g.q[pick].cpu(), type(g.cache)(*(t[g.slot_ids[pick].long()].cpu() for t in
                                          (g.cache.k, g.cache.v, g.cache.k_scale,
                                           g.cache.v_scale, g.cache.k_calibration))),
        g.cached_lens[pick].cpu(), torch.arange(len(pick), dtype=torch.int32),
        torch.tensor([len(pick)], dtype=torch.int32), [ctx[i] for i in pick])
    assert_attn_close(o[pick], oracle_out(sub), "headline sampled")


def test_decode_through_c_abi(ie, workloads, dev, native):
    """The same computation driven through libie_attn.so's C entry point directly."""
    ctx = [300, 2000, 77]
    wl = workloads.decode_workload(ctx, seed=13)
    ref = oracle_out(wl)
    g = wl.to(dev)
    lib = native.cabi()
    ws_bytes = lib.ie_decode_attention_workspace_size(len(ctx), 16, 128)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    out = torch.empty(len(ctx), 16, 128, dtype=torch.bfloat16, device=dev)
    desc = native.KVCacheDesc.of(g.cache)
    fn = lib.ie_decode_attention
    fn.restype = ctypes.c_int
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = fn(p(g.q), ctypes.c_int64(g.q.stride(0)), ctypes.c_int64(g.q.stride(1)),
            ctypes.c_int32(len(ctx)), ctypes.c_int32(16), ctypes.byref(desc), p(g.cached_lens),
            p(g.slot_ids), p(g.num_decoding), ctypes.c_float(SCALE), p(out),
            ctypes.c_int64(out.stride(0)), ctypes.c_int64(out.stride(1)), p(ws),
            ctypes.c_size_t(ws_bytes),
            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, lib.ie_attn_last_error()
    torch.cuda.synchronize()
    assert_attn_close(bf16_np(out), ref, "c-abi decode")


def test_decode_split_count_invariance(ie, workloads, dev):
    """Different batch mixes change the piece size; a sequence's output must not depend on it
    beyond tolerance: the same 3 sequences alone vs. next to 60 long ones."""
    wl = workloads.decode_workload([4000, 1000, 130] + [4096] * 60, seed=17)
    g = wl.to(dev)
    out_all = ie.decode_attention(g.q, g.cache, g.cached_lens, g.slot_ids, g.num_decoding, SCALE)
    nd3 = torch.tensor([3], dtype=torch.int32, device=dev)
    out3 = torch.zeros_like(out_all)
    ie.decode_attention(g.q, g.cache, g.cached_lens, g.slot_ids, nd3, SCALE, out=out3)
    torch.cuda.synchronize()
    a, b = bf16_np(out_all[:3]), bf16_np(out3[:3])
    assert np.abs(a - b).max() <= 1e-2
