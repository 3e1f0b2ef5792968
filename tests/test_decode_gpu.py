"""Split-K decode attention on the GPU against the oracle (bf16 tolerance), through the torch
op and through the C ABI, at BASELINE configs 1-3 and ragged edge cases."""

import ctypes

import numpy as np
import pytest
import torch

from helpers import TOL_MAX, TOL_MEAN, assert_attn_close, bf16_np, cache_np, rel_err, say
from oracle import attention as oat
from oracle import work_split as ows

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


def test_decode_workspace_reuse_across_batches(ie, workloads, dev):
    """The op keeps one zeroed workspace per stream whose arrival counts every call leaves at
    zero: calls of growing, shrinking and above-1024 batches in a row, each against the oracle.
    A count region that moved with the batch would let one call's partials land on the next
    call's counts."""
    rng = np.random.default_rng(17)
    plan = [[20000], [3000] * 64, [64] * 40 + [9000], [int(x) for x in rng.integers(1, 200, 1100)],
            [5, 4000, 70], [int(x) for x in rng.integers(1, 200, 1100)], [33000, 2]]
    for i, ctx in enumerate(plan):
        say(f"decode workspace reuse call {i}: B={len(ctx)} max ctx {max(ctx)}")
        wl = workloads.decode_workload(ctx, seed=100 + i, pool=len(ctx) + 3)
        ref = oracle_out(wl)
        g = wl.to(dev)
        out = ie.decode_attention(g.q, g.cache, g.cached_lens, g.slot_ids, g.num_decoding, SCALE)
        torch.cuda.synchronize()
        assert_attn_close(bf16_np(out), ref, f"reuse call {i} B={len(ctx)}")


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


def sampled_check(ie, workloads, dev, ctx, pick, seed, what, **kw):
    """The batch generated on the GPU, decoded whole; all outputs finite, and the sequences
    `pick` checked against the oracle on their own cache rows."""
    g = workloads.decode_workload(ctx, seed=seed, device=dev, **kw)
    out = ie.decode_attention(g.q, g.cache, g.cached_lens, g.slot_ids, g.num_decoding, SCALE)
    torch.cuda.synchronize()
    nd = int(g.num_decoding[0])
    o = bf16_np(out)
    assert np.isfinite(o[:nd]).all()
    sub = workloads.DecodeWorkload(
        g.q[pick].cpu(), type(g.cache)(*(t[g.slot_ids[pick].long()].cpu() for t in
                                          (g.cache.k, g.cache.v, g.cache.k_scale,
                                           g.cache.v_scale, g.cache.k_calibration))),
        g.cached_lens[pick].cpu(), torch.arange(len(pick), dtype=torch.int32),
        torch.tensor([len(pick)], dtype=torch.int32), [ctx[i] for i in pick])
    assert_attn_close(o[pick], oracle_out(sub), what)
    del g, out
    torch.cuda.empty_cache()


@pytest.mark.parametrize("B,ctx", [(64, 4096), (16, 4096), (256, 1024), (256, 4096)])
def test_decode_config3_sampled(ie, workloads, dev, B, ctx):
    """BASELINE config 3 points at full size, generated on the GPU (B=64 ctx=4096 is the
    headline, 8-wave workgroups; B=256 runs 2-wave workgroups, whose per-head target of 256
    holds the batch): 8 sampled sequences checked against the oracle."""
    say(f"decode config 3 B={B} ctx={ctx} (sampled)")
    pick = sorted({0, 1, B // 4, B // 2 - 1, B // 2, 3 * B // 4, B - 2, B - 1})
    sampled_check(ie, workloads, dev, [ctx] * B, pick, seed=B + ctx, what=f"config3 {B}x{ctx}")


@pytest.mark.parametrize("B,nd,lo,hi,seed", [
    (200, 170, 1, 3000, 31),  # 2-wave workgroups (target 256 on 256 CUs), fitted pieces
    (300, 299, 1, 600, 32),   # above every target: the reference's TARGET + B grid
    (65, 65, 2000, 9000, 33),  # one past the 8-wave target: 4-wave workgroups, several splits
])
def test_decode_ragged_large_batch(ie, workloads, dev, B, nd, lo, hi, seed):
    """Batches above the 8-wave workgroups' per-head target (64 on 256 CUs) with
    num_decoding < B: 4- and 2-wave workgroups with fitted pieces, and above every target the
    reference's unfitted piece rule and TARGET + B grid (kernels.py:294-314); every decoding row
    against the oracle and the rows past num_decoding untouched."""
    ctx = [int(x) for x in np.random.default_rng(seed).integers(lo, hi + 1, B)]
    say(f"decode ragged B={B} num_decoding={nd} ctx {min(ctx)}..{max(ctx)}")
    wl = workloads.decode_workload(ctx, seed=seed, num_decoding=nd)
    ref = oracle_out(wl, nd=nd)
    g = wl.to(dev)
    out = torch.full((B, 16, 128), 3.0, dtype=torch.bfloat16, device=dev)
    ie.decode_attention(g.q, g.cache, g.cached_lens, g.slot_ids, g.num_decoding, SCALE, out=out)
    torch.cuda.synchronize()
    o = bf16_np(out)
    assert_attn_close(o[:nd], ref[:nd], f"ragged large B={B}")
    assert np.all(o[nd:] == 3.0)


def test_decode_long_and_short_mix_above_target(ie, workloads, dev):
    """96 sequences, 6 of them 30-60K tokens long (4-wave workgroups): the long ones split into
    many pieces, merged by their last piece."""
    rng = np.random.default_rng(41)
    ctx = [int(x) for x in rng.integers(100, 500, 90)] + [int(x) for x in
                                                          rng.integers(30000, 60000, 6)]
    rng.shuffle(ctx)
    say(f"decode long/short mix B={len(ctx)} max ctx {max(ctx)}")
    wl = workloads.decode_workload(ctx, seed=41)
    ref = oracle_out(wl)
    g = wl.to(dev)
    out = ie.decode_attention(g.q, g.cache, g.cached_lens, g.slot_ids, g.num_decoding, SCALE)
    torch.cuda.synchronize()
    assert_attn_close(bf16_np(out), ref, "long/short mix")


@pytest.mark.parametrize("v_mult,sink", [(1e-2, 0.8), (1e-4, 0.8), (1e2, 0.8), (1e-2, 0.0),
                                         (1.0, 0.8)])
def test_decode_v_magnitude_and_sink(ie, workloads, dev, v_mult, sink):
    """V far from unit scale, with an attention sink (one key scoring ~9 above the rest, so the
    thousands of tail keys each weigh ~1e-4 and together about as much as the sink): the
    products p * v_scale span many binades, and the scale-normalised error must stay within
    the bf16 tolerance whatever V's magnitude."""
    ctx = [8000, 6000, 9000, 3000]
    wl = workloads.decode_workload(ctx, seed=51, v_mult=v_mult, sink_alpha=sink)
    ref = oracle_out(wl)
    g = wl.to(dev)
    out = ie.decode_attention(g.q, g.cache, g.cached_lens, g.slot_ids, g.num_decoding, SCALE)
    torch.cuda.synchronize()
    o = bf16_np(out)
    r = rel_err(o, ref)
    say(f"v_mult {v_mult} sink {sink}: scaled max err {r.max():.3e} mean {r.mean():.3e}")
    assert np.isfinite(o).all()
    assert r.max() <= TOL_MAX and r.mean() <= TOL_MEAN


@pytest.mark.parametrize("ctx,nd", [
    ([4096] * 64, 64), ([4096] * 63 + [1], 64), ([7] * 10, 10), ([100, 3000, 5] * 7, 20),
    ([int(x) for x in np.random.default_rng(3).integers(1, 5000, 64)], 64),
    ([int(x) for x in np.random.default_rng(4).integers(1, 5000, 200)], 170),
    ([1024] * 256, 256), ([200] * 90 + [50000] * 6, 96), ([33000], 1), ([5, 6], 0),
    ([int(x) for x in np.random.default_rng(5).integers(1, 600, 300)], 299),
])
def test_decode_plan_matches_oracle(ie, native, dev, ctx, nd):
    """The decode launch's work list, as the device computes it (ie_decode_attention_plan runs
    the decode kernel's own assignment code), equals oracle/work_split.decode_work_plan entry
    for entry, and no piece of the oracle's list falls outside the launch's grid."""
    lib = native.cabi()
    B = len(ctx)
    hkv = 8
    target = lib.ie_decode_attention_target(ctypes.c_int32(B), ctypes.c_int32(hkv))
    grid = lib.ie_decode_attention_grid(ctypes.c_int32(B), ctypes.c_int32(hkv))
    assert grid == (target if B <= target else target + B)
    cl = torch.tensor([c - 1 for c in ctx], dtype=torch.int32, device=dev)
    ndt = torch.tensor([nd], dtype=torch.int32, device=dev)
    rows = torch.full((grid, 4), -7, dtype=torch.int32, device=dev)
    fn = lib.ie_decode_attention_plan
    fn.restype = ctypes.c_int
    rc = fn(ctypes.c_void_p(cl.data_ptr()), ctypes.c_void_p(ndt.data_ptr()), ctypes.c_int32(B),
            ctypes.c_int32(hkv), ctypes.c_void_p(rows.data_ptr()),
            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, lib.ie_attn_last_error()
    torch.cuda.synchronize()
    got = rows.cpu().numpy()
    piece, ref_rows = ows.decode_work_plan(np.array(ctx) - 1, nd, B, target, min_piece=128)
    ref = np.array(ref_rows)
    say(f"plan B={B} nd={nd}: piece {piece}, {int((ref[:, 2] > 0).sum())} work entries, "
        f"grid {grid}")
    assert np.all(ref[grid:, 2] == 0), "oracle pieces past the grid"
    if nd > 0:
        assert np.all(got[:, 3] == piece)
    work = ref[:grid, 2] > 0
    assert np.array_equal(got[:, 2] > 0, work)
    assert np.array_equal(got[work, :3], ref[:grid][work])


def test_decode_through_c_abi(ie, workloads, dev, native):
    """The same computation driven through libie_attn.so's C entry point directly, three times
    on one workspace: the sequences of 300 and 2,000 tokens split into pieces that the last one
    to finish merges, and every call leaves the workspace's arrival counts at zero again."""
    ctx = [300, 2000, 77]
    wl = workloads.decode_workload(ctx, seed=13)
    ref = oracle_out(wl)
    g = wl.to(dev)
    lib = native.cabi()
    ws_bytes = lib.ie_decode_attention_workspace_size(len(ctx), 16, 128)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)  # arrival counts start at 0
    out = torch.empty(len(ctx), 16, 128, dtype=torch.bfloat16, device=dev)
    desc = native.KVCacheDesc.of(g.cache)
    fn = lib.ie_decode_attention
    fn.restype = ctypes.c_int
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    first = None
    for call in range(3):
        out.fill_(9.0)
        rc = fn(p(g.q), ctypes.c_int64(g.q.stride(0)), ctypes.c_int64(g.q.stride(1)),
                ctypes.c_int32(len(ctx)), ctypes.c_int32(16), ctypes.byref(desc),
                p(g.cached_lens), p(g.slot_ids), p(g.num_decoding), ctypes.c_float(SCALE),
                p(out), ctypes.c_int64(out.stride(0)), ctypes.c_int64(out.stride(1)), p(ws),
                ctypes.c_size_t(ws_bytes),
                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        assert rc == 0, lib.ie_attn_last_error()
        torch.cuda.synchronize()
        assert not ws[:len(ctx) * 8 * 4].any(), f"call {call} left arrival counts behind"
        if first is None:
            first = out.clone()
            assert_attn_close(bf16_np(out), ref, "c-abi decode")
        else:
            assert torch.equal(out, first), f"call {call} differs from the first"


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
