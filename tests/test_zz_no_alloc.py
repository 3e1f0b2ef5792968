"""ie_decode_attention_noalloc (the decode entry point that allocates nothing, its workspace
in a static device array) against ie_decode_attention with a caller workspace, through the C
ABI: identical bits on two calls in a row, the second with a smaller batch, and the host-side
rejection of a batch above the 1024 sequences the array serves."""

import ctypes

import numpy as np
import pytest
import torch

from helpers import say

pytestmark = pytest.mark.gpu
SCALE = 128 ** -0.5


def _call(lib, native, g, out, ws=None):
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    desc = native.KVCacheDesc.of(g.cache)
    B, hq = g.q.shape[0], g.q.shape[1]
    args = [p(g.q), ctypes.c_int64(g.q.stride(0)), ctypes.c_int64(g.q.stride(1)),
            ctypes.c_int32(B), ctypes.c_int32(hq), ctypes.byref(desc), p(g.cached_lens),
            p(g.slot_ids), p(g.num_decoding), ctypes.c_float(SCALE), p(out),
            ctypes.c_int64(out.stride(0)), ctypes.c_int64(out.stride(1))]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if ws is None:
        fn = lib.ie_decode_attention_noalloc
        fn.restype = ctypes.c_int
        rc = fn(*args, stream)
    else:
        fn = lib.ie_decode_attention
        fn.restype = ctypes.c_int
        rc = fn(*args, p(ws), ctypes.c_size_t(ws.numel()), stream)
    assert rc == 0, lib.ie_attn_last_error()


@pytest.mark.parametrize("hq,hkv", [(16, 8), (32, 8), (40, 8), (2, 1)])
def test_noalloc_matches_workspace_entry(ie, workloads, native, dev, hq, hkv):
    lib = native.cabi()
    lib.ie_decode_attention_noalloc_max_bytes.restype = ctypes.c_size_t
    lib.ie_decode_attention_workspace_size.restype = ctypes.c_size_t
    cap = lib.ie_decode_attention_noalloc_max_bytes()
    assert cap == 16 << 20
    # two calls in a row, the second with a smaller batch: the first call's plan and partials
    # are still in the array when the second runs (any head geometry: the count region is laid
    # out per query head)
    for ctx, seed in (([3000, 40, 9000, 128, 1, 4096] * 12 + [20000], 61),
                      ([700, 2, 5000], 62)):
        B = len(ctx)
        say(f"noalloc decode hq={hq} hkv={hkv} B={B} max ctx {max(ctx)}")
        g = workloads.decode_workload(ctx, seed=seed, device=dev, hq=hq, hkv=hkv)
        ws_bytes = lib.ie_decode_attention_workspace_size(B, hq, 128)
        assert ws_bytes <= cap
        ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)  # arrival counts start at 0
        ref = torch.full((B, hq, 128), 5.0, dtype=torch.bfloat16, device=dev)
        got = torch.full((B, hq, 128), 6.0, dtype=torch.bfloat16, device=dev)
        _call(lib, native, g, ref, ws)
        _call(lib, native, g, got)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), \
            "no-alloc output differs from the workspace entry point"


def test_noalloc_rejects_batch_beyond_scratch(ie, native, dev):
    lib = native.cabi()
    cap = lib.ie_decode_attention_noalloc_max_bytes()
    B = 1
    while lib.ie_decode_attention_workspace_size(B, 16, 128) <= cap:
        B *= 2
    c = ie.make_layer_cache(2, 8, 128, 128, device=dev)
    q = torch.zeros(B, 16, 128, dtype=torch.bfloat16, device=dev)
    i = torch.zeros(B, dtype=torch.int32, device=dev)
    nd = torch.zeros(1, dtype=torch.int32, device=dev)
    out = torch.zeros_like(q)
    desc = native.KVCacheDesc.of(c)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    fn = lib.ie_decode_attention_noalloc
    fn.restype = ctypes.c_int
    rc = fn(p(q), ctypes.c_int64(2048), ctypes.c_int64(128), ctypes.c_int32(B),
            ctypes.c_int32(16), ctypes.byref(desc), p(i), p(i), p(nd), ctypes.c_float(SCALE),
            p(out), ctypes.c_int64(2048), ctypes.c_int64(128),
            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 1 and b"no-alloc" in lib.ie_attn_last_error()
    # a batch just above the 1024 sequences that share the array's count region
    B = 1025
    q = torch.zeros(B, 16, 128, dtype=torch.bfloat16, device=dev)
    i = torch.zeros(B, dtype=torch.int32, device=dev)
    out2 = torch.zeros_like(q)
    rc = fn(p(q), ctypes.c_int64(2048), ctypes.c_int64(128), ctypes.c_int32(B),
            ctypes.c_int32(16), ctypes.byref(desc), p(i), p(i), p(nd), ctypes.c_float(SCALE),
            p(out2), ctypes.c_int64(2048), ctypes.c_int64(128),
            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 1 and b"no-alloc" in lib.ie_attn_last_error()
    torch.cuda.synchronize()
    assert not out.any() and not out2.any()
