"""Chunked-prefill attention on the GPU (int8 prefix dequantized in LDS, bf16 MFMA) against the
oracle (reference rounding: bf16 prefix, bf16 P) within bf16 tolerance."""

import numpy as np
import pytest
import torch

from helpers import assert_attn_close, bf16_np, cache_np, say
from oracle import attention as oat
from oracle import kv_cache as okv

pytestmark = pytest.mark.gpu


def oracle_prefill(wl):
    ins = {n: t.cpu().numpy() for n, t in wl.inputs.items()}
    kp, vp = okv.dequantize_kv_prefix(cache_np(wl.cache), ins["cu_cached"], ins["slot_ids"])
    return oat.prefill_attention(bf16_np(wl.q), bf16_np(wl.k), bf16_np(wl.v), ins["cu_seqlens"],
                                 ins["tile_start"], wl.block_m, kp, vp, ins["cu_cached"])


def run_gpu(ie, wl):
    gi = wl.inputs
    return ie.prefill_attention(wl.q, wl.k, wl.v, gi["seq_ids"], gi["cu_seqlens"],
                                gi["tile_start"], wl.cache, gi["slot_ids"], gi["cu_cached"],
                                wl.block_m)


def check(ie, workloads, wl, dev, what):
    ref = oracle_prefill(wl)
    g = workloads.mixed_to(wl, dev)
    out = run_gpu(ie, g)
    torch.cuda.synchronize()
    cov = ~np.isnan(ref[:, 0, 0])
    assert cov.any()
    assert_attn_close(bf16_np(out)[cov], ref[cov], what)


def test_prefill_config4(ie, workloads, dev):
    say("prefill config 4 (30 decoders, 512 new + 0 cached, 512 new + 1536 cached)")
    check(ie, workloads, workloads.config4(seed=2), dev, "prefill config4")


@pytest.mark.parametrize("block_m", [16, 32, 64, 128, 192])
def test_prefill_tile_sizes(ie, workloads, dev, block_m):
    say(f"prefill block_m={block_m}")
    wl = workloads.mixed_workload([7, 300], [(100, 0), (65, 77), (1, 130), (129, 1)], seed=3,
                                  block_m=block_m, max_len=1024)
    check(ie, workloads, wl, dev, f"prefill block_m={block_m}")


@pytest.mark.parametrize("chunks", [
    [(1, 0)], [(64, 0)], [(63, 64)], [(200, 1000)], [(3, 0), (0, 0), (5, 5)], [(700, 2047)],
])
def test_prefill_edges(ie, workloads, dev, chunks):
    say(f"prefill edge chunks {chunks}")
    wl = workloads.mixed_workload([], chunks, seed=len(chunks), block_m=128, max_len=4096)
    check(ie, workloads, wl, dev, f"prefill {chunks}")


@pytest.mark.parametrize("chunks", [[(2048, 2048)] * 4, [(1024, 7168)] * 4])
def test_prefill_long_sampled(ie, workloads, dev, chunks):
    """The long-prefill shapes the benchmark times (4 x 2048 new after 2048 cached, 4 x 1024 new
    after 7168): every row finite, and rows at the chunk edges, tile and sub-block boundaries
    and inside checked against the oracle."""
    say(f"prefill long {chunks} (sampled rows)")
    max_len = max(L + c for L, c in chunks)
    wl = workloads.mixed_workload([], chunks, seed=21, block_m=128, max_len=max_len)
    cu = wl.inputs["cu_seqlens"].numpy()
    rows = []
    for e in range(len(chunks)):
        L = chunks[e][0]
        rows += [int(cu[e]) + o for o in (0, 1, 63, 64, 127, 128, 129, L // 2, L - 65, L - 1)]
    ins = {n: t.numpy() for n, t in wl.inputs.items()}
    kp, vp = okv.dequantize_kv_prefix(cache_np(wl.cache), ins["cu_cached"], ins["slot_ids"])
    ref = oat.prefill_attention(bf16_np(wl.q), bf16_np(wl.k), bf16_np(wl.v), ins["cu_seqlens"],
                                ins["tile_start"], wl.block_m, kp, vp, ins["cu_cached"],
                                rows=rows)
    g = workloads.mixed_to(wl, dev)
    out = run_gpu(ie, g)
    torch.cuda.synchronize()
    o = bf16_np(out)
    assert np.isfinite(o).all()
    assert_attn_close(o[rows], ref[rows], f"prefill long {chunks[0]} x {len(chunks)}")


@pytest.mark.parametrize("chunks", [
    [(64, 1000 + 250 * i) for i in range(16)],
    [((33, 64, 100, 128)[i % 4], 500 + 175 * i) for i in range(20)],
])
def test_prefill_straddling_pieces(ie, workloads, dev, chunks):
    """A few short chunks over long prefixes: 16 or 20 sub-blocks, each with prefix and chunk
    tiles, i.e. (sub-block, KV head) pairs that fit a 256-CU device's slots one piece each, while
    their prefix and chunk parts do not. The launch then splits each pair into even ranges of
    its tiles, the range crossing into the chunk running both loops. Every row finite; the
    first, second, middle and last rows of every chunk against the oracle (every piece of a
    pair adds keys to every row of its sub-block)."""
    say(f"prefill straddling pieces, {len(chunks)} chunks")
    max_len = max(L + c for L, c in chunks)
    wl = workloads.mixed_workload([], chunks, seed=31, block_m=128, max_len=max_len)
    cu = wl.inputs["cu_seqlens"].numpy()
    rows = sorted({int(cu[e]) + o for e, (L, _) in enumerate(chunks) for o in (0, 1, L // 2, L - 1)})
    ins = {n: t.numpy() for n, t in wl.inputs.items()}
    kp, vp = okv.dequantize_kv_prefix(cache_np(wl.cache), ins["cu_cached"], ins["slot_ids"])
    ref = oat.prefill_attention(bf16_np(wl.q), bf16_np(wl.k), bf16_np(wl.v), ins["cu_seqlens"],
                                ins["tile_start"], wl.block_m, kp, vp, ins["cu_cached"],
                                rows=rows)
    out = run_gpu(ie, workloads.mixed_to(wl, dev))
    torch.cuda.synchronize()
    o = bf16_np(out)
    assert np.isfinite(o).all()
    assert_attn_close(o[rows], ref[rows], f"prefill straddling {len(chunks)} chunks")


@pytest.mark.parametrize("chunks", [[(512, 0), (512, 1536)], [(300, 5000), (64, 9000)],
                                    [(64, 1000 + 250 * i) for i in range(16)]])
def test_prefill_split_merge_fallback(ie, workloads, dev, monkeypatch, chunks):
    """Split pieces wait a bounded time for their pair's other pieces and then merge a share
    each; a piece that gives up leaves its share to the last one to finish. With the wait set to
    zero every piece but the last gives up, so the last finisher merges every share: the output
    must be bit-identical to the cooperative merge, and the next calls (the counters left at
    zero) too."""
    say(f"prefill split-merge fallback {chunks}")
    wl = workloads.mixed_to(workloads.mixed_workload([], chunks, seed=5, block_m=128,
                                                     max_len=10240), dev)
    monkeypatch.delenv("IE_PREFILL_MERGE_WAIT_US", raising=False)
    coop = run_gpu(ie, wl)
    monkeypatch.setenv("IE_PREFILL_MERGE_WAIT_US", "0")
    fall = [run_gpu(ie, wl) for _ in range(3)]
    monkeypatch.delenv("IE_PREFILL_MERGE_WAIT_US")
    again = run_gpu(ie, wl)
    torch.cuda.synchronize()
    for i, f in enumerate(fall):
        assert torch.equal(f.view(torch.int16), coop.view(torch.int16)), f"fallback call {i}"
    assert torch.equal(again.view(torch.int16), coop.view(torch.int16))


@pytest.mark.parametrize("seed", range(6))
def test_prefill_random_steps(ie, workloads, dev, seed):
    """Seeded random mixed steps (decoders, 1-4 chunks of 1-320 new tokens over 0-1,500 cached,
    block_m 64 or 128): whichever of the unsplit, separate-split and straddling forms the launch
    takes, and with workgroups past the slots, every prefill row matches the oracle."""
    rng = np.random.default_rng(100 + seed)
    decoders = [int(x) for x in rng.integers(1, 1500, int(rng.integers(0, 40)))]
    chunks = [(int(rng.integers(1, 321)), 0 if rng.random() < 0.3 else int(rng.integers(1, 1501)))
              for _ in range(int(rng.integers(1, 5)))]
    block_m = int(rng.choice([64, 128]))
    say(f"prefill random step seed {seed}: {len(decoders)} decoders, chunks {chunks}, "
        f"block_m {block_m}")
    wl = workloads.mixed_workload(decoders, chunks, seed=seed, block_m=block_m, max_len=2048)
    check(ie, workloads, wl, dev, f"prefill random step {seed}")
