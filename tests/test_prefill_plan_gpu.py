"""prefill_attention with its work list computed once per step (prefill_plan, then
ie_prefill_attention_planned): outputs bit for bit equal to the launch that derives the list
from the tile metadata itself, on config 4, on long prefixes whose pieces straddle the prefix
and the chunk, at GQA 5 (40/8 heads: an odd ratio's one-head unit), with more entries than the
kernel stages on chip, for two layers that share one plan, inside a replayed hipGraph, and through
the attention layer. The self-scheduling launch is the one the oracle tests pin
(test_prefill_gpu.py, test_prefill_peaked_gpu.py); here one config-4 case is also checked
against the oracle directly.
"""

import importlib

import numpy as np
import pytest
import torch

from helpers import PLAN_FIELDS, assert_attn_close, bf16_np, cache_np, prefill_plan, say
from oracle import attention as oat
from oracle import kv_cache as okv

pytestmark = pytest.mark.gpu
F = {n: i for i, n in enumerate(PLAN_FIELDS)}


def _run(K, g, plan=None, q=None):
    gi = g.inputs
    return K.prefill_attention(g.q if q is None else q, g.k, g.v, gi["seq_ids"],
                               gi["cu_seqlens"], gi["tile_start"], g.cache, gi["slot_ids"],
                               gi["cu_cached"], g.block_m, plan)


def _plan(K, g):
    gi = g.inputs
    return K.prefill_plan(gi["seq_ids"], gi["cu_seqlens"], gi["tile_start"], gi["slot_ids"],
                          gi["cu_cached"], g.q.shape[0], g.q.shape[1], g.cache.k.shape[1],
                          g.block_m)


def _covered(rows, n):
    """Packed rows some workgroup of the launch writes (the outputs of rows no tile covers, such
    as the decoders' rows of a mixed step, are left untouched)."""
    cov = np.zeros(n, dtype=bool)
    for r in rows[rows[:, F["found"]] == 1]:
        cov[r[F["r0"]]:r[F["r1"]]] = True
    return torch.from_numpy(cov)


def _workload(workloads, case):
    if case == "config4":
        return workloads.config4(seed=31)
    if case == "straddle":  # 4 x 512 new after 8192 cached: pieces cross into the chunk
        return workloads.mixed_workload([], [(512, 8192)] * 4, seed=32, block_m=128,
                                        max_len=8704)
    if case == "gqa5":
        return workloads.mixed_workload([7, 40], [(200, 300), (129, 1000)], seed=33,
                                        block_m=128, max_len=1216, hq=40, hkv=8)
    if case == "many_entries":  # 600 entries: the entry of a tile read from seq_ids
        return workloads.mixed_workload([5] * 597, [(300, 0), (100, 700), (64, 64)], seed=34,
                                        block_m=64, max_len=1024)
    raise ValueError(case)


@pytest.mark.parametrize("case", ["config4", "straddle", "gqa5", "many_entries"])
def test_planned_prefill_equals_self_scheduled(ie, workloads, native, dev, case):
    K = ie.kernels
    say(f"planned prefill: {case}")
    g = workloads.mixed_to(_workload(workloads, case), dev)
    plan = _plan(K, g)
    torch.cuda.synchronize()
    # the op's plan is the export the C ABI writes (tests read its fields elsewhere)
    assert np.array_equal(plan.cpu().numpy(), prefill_plan(native, g))
    rows = plan.cpu().numpy()
    slots = g.inputs["slot_ids"].cpu().numpy()
    cu = g.inputs["cu_seqlens"].cpu().numpy()
    for r in rows[rows[:, F["found"]] == 1]:
        e = int(np.searchsorted(cu, r[F["seq_start"]], side="right")) - 1
        assert cu[e] == r[F["seq_start"]] and r[F["slot"]] == slots[e], "plan slot field"
    base = _run(K, g)
    planned = _run(K, g, plan)
    torch.cuda.synchronize()
    cov = _covered(rows, g.q.shape[0])
    assert cov.sum() > 0
    assert torch.equal(base[cov], planned[cov]), f"{case}: planned launch differs"


def test_planned_prefill_config4_against_oracle(ie, workloads, dev):
    K = ie.kernels
    wl = workloads.config4(seed=35)
    ins = {n: t.numpy() for n, t in wl.inputs.items()}
    kp, vp = okv.dequantize_kv_prefix(cache_np(wl.cache), ins["cu_cached"], ins["slot_ids"])
    ref = oat.prefill_attention(bf16_np(wl.q), bf16_np(wl.k), bf16_np(wl.v), ins["cu_seqlens"],
                                ins["tile_start"], wl.block_m, kp, vp, ins["cu_cached"])
    g = workloads.mixed_to(wl, dev)
    out = _run(K, g, _plan(K, g))
    torch.cuda.synchronize()
    cov = ~np.isnan(ref[:, 0, 0])
    assert_attn_close(bf16_np(out)[cov], ref[cov], "planned prefill config 4")


def test_one_plan_serves_two_layers(ie, workloads, dev):
    """Two layers of one step: different q/k/v and caches, the same metadata and plan."""
    K = ie.kernels
    g1 = workloads.mixed_to(workloads.config4(seed=36), dev)
    g2 = workloads.mixed_to(workloads.config4(seed=37), dev)
    for n in ("seq_ids", "cu_seqlens", "tile_start", "slot_ids", "cu_cached"):
        assert torch.equal(g1.inputs[n], g2.inputs[n])
    plan = _plan(K, g1)
    cov = _covered(plan.cpu().numpy(), g1.q.shape[0])
    for g in (g1, g2):
        assert torch.equal(_run(K, g)[cov], _run(K, g, plan)[cov])


def test_planned_prefill_in_graph(ie, workloads, dev):
    """The plan computed in the graph once, the prefill launch run twice from it, replayed three
    times with new q in between: every replay equals the eager self-scheduled launch."""
    K = ie.kernels
    g = workloads.mixed_to(workloads.config4(seed=38), dev)
    q = g.q.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        _run(K, g, _plan(K, g), q)  # warm-up on the capture stream: its workspace exists
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        plan = _plan(K, g)
        o1 = _run(K, g, plan, q)
        o2 = _run(K, g, plan, q)
    cov = _covered(_plan(K, g).cpu().numpy(), q.shape[0])
    gen = torch.Generator().manual_seed(39)
    for rep in range(3):
        q.copy_(torch.randn(q.shape, generator=gen).bfloat16().to(dev))
        graph.replay()
        torch.cuda.synchronize()
        ref = _run(K, g, None, q)
        torch.cuda.synchronize()
        assert torch.equal(o1[cov], ref[cov]) and torch.equal(o2[cov], ref[cov]), f"replay {rep}"


def test_attention_layer_with_plan(ie, workloads, dev):
    """The attention layer's step with prefill_plan and decode_plan: the same output and cache
    bits."""
    ms = importlib.import_module("test_mixed_step_gpu")
    K = ie.kernels
    wl = workloads.config4(seed=40)
    al, g, _, q, k, v, qw, kw, cos, sin = ms.step_setup(workloads, wl, dev, 41)
    g2 = workloads.mixed_to(wl, dev)
    gi = g.inputs
    plan = _plan(K, g)
    out = ms.run_step(al, g, q, k, v, qw, kw, cos, sin)
    gi2 = g2.inputs
    out2 = al.attention(q, k, v, gi2["seq_ids"], gi2["cu_seqlens"], cos, sin, g2.cache,
                        gi2["cached_lens"], gi2["slot_ids"], gi2["tile_start"], g2.block_m,
                        al.PrefixScratch(None, None, gi2["cu_cached"]), gi2["num_decoding"], qw,
                        kw, ms.EPS, prefill_plan=plan,
                        decode_plan=K.decode_plan(gi2["cached_lens"], gi2["num_decoding"],
                                                  gi2["slot_ids"].shape[0], 16, 8))
    torch.cuda.synchronize()
    assert torch.equal(out, out2)
    for a, b in zip((g.cache.k, g.cache.v, g.cache.k_scale, g.cache.v_scale,
                     g.cache.k_calibration),
                    (g2.cache.k, g2.cache.v, g2.cache.k_scale, g2.cache.v_scale,
                     g2.cache.k_calibration)):
        assert torch.equal(a, b)
    del gi
