"""Pins the oracle's decode / prefill attention against float64 torch SDPA (an independent library
routine), split-K invariance and brute force on tiny shapes (CPU only)."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oat
from oracle import kv_cache as okv
from oracle import work_split as ows

TOL_MAX, TOL_MEAN = 2e-2, 2e-3  # BASELINE north_star tolerances for bf16 attention outputs


def cache_np(c):
    return okv.CacheArrays(c.k.numpy(), c.v.numpy(), c.k_scale.numpy(), c.v_scale.numpy(),
                           c.k_calibration.numpy())


def sdpa_decode64(wl):
    """torch SDPA in float64 over the dequantized cache, GQA expanded explicitly."""
    q = wl.q.double()
    out = torch.full(q.shape, float("nan"), dtype=torch.float64)
    c = wl.cache
    for b, ctx in enumerate(wl.ctx):
        s = int(wl.slot_ids[b])
        k = c.k[s, :, :ctx].double() * c.k_scale[s, :, :ctx, None].double()
        v = c.v[s, :, :ctx].double() * c.v_scale[s, :, :ctx, None].double()
        k = k.repeat_interleave(2, dim=0)  # [Hq, ctx, D]
        v = v.repeat_interleave(2, dim=0)
        out[b] = F.scaled_dot_product_attention(q[b][:, None], k, v, scale=128 ** -0.5)[:, 0]
    return out.numpy()


@pytest.mark.parametrize("cfg", ["1", "2", "3:4:700"])
def test_decode_oracle_vs_sdpa64(workloads, cfg):
    wl = workloads.decode_workload(workloads.decode_ctx_lens(cfg), seed=11)
    ref = sdpa_decode64(wl)
    cn = cache_np(wl.cache)
    q = wl.q.float().numpy()
    f64 = oat.decode_attention_f64(q, cn, wl.cached_lens.numpy(), wl.slot_ids.numpy(),
                                   len(wl.ctx), 128 ** -0.5)
    assert np.abs(f64 - ref).max() < 1e-10
    mirror = oat.decode_attention(q, cn, wl.cached_lens.numpy(), wl.slot_ids.numpy(),
                                  len(wl.ctx), 128 ** -0.5)
    err = np.abs(mirror - ref)
    assert err.max() < 4e-3 and err.mean() < 5e-4


def test_decode_oracle_split_invariance_and_untouched_rows(workloads):
    wl = workloads.decode_workload([300, 129, 64, 1000], seed=3)
    cn = cache_np(wl.cache)
    q = wl.q.float().numpy()
    args = (q, cn, wl.cached_lens.numpy(), wl.slot_ids.numpy(), 3, 128 ** -0.5)
    one = oat.decode_attention(*args)
    piece = 128
    splits = [[(a, min(a + piece, c)) for a in range(0, c, piece)] for c in wl.ctx]
    many = oat.decode_attention(*args, splits=splits)
    assert np.isnan(one[3]).all() and np.isnan(many[3]).all()
    err = np.abs(one[:3] - many[:3])
    assert err.max() < 4e-3


def test_decode_oracle_catches_wrong_head_mapping(workloads):
    """A planted GQA mistake (q head h reading kv head h % Hkv) must fail the SDPA check."""
    wl = workloads.decode_workload([200, 200], seed=5)
    ref = sdpa_decode64(wl)
    cn = cache_np(wl.cache)
    cn_bad = cn.copy()
    cn_bad.k = cn.k[:, [0, 4, 1, 5, 2, 6, 3, 7]]  # permute kv heads
    bad = oat.decode_attention(wl.q.float().numpy(), cn_bad, wl.cached_lens.numpy(),
                               wl.slot_ids.numpy(), 2, 128 ** -0.5)
    assert np.abs(bad - ref).max() > TOL_MAX


def sdpa_prefill64(wl, kp, vp):
    """float64 SDPA of every covered packed row against [prefix || causal chunk]."""
    cu = wl.inputs["cu_seqlens"].numpy()
    cc = wl.inputs["cu_cached"].numpy()
    covered = oat.prefill_rows(cu, wl.inputs["tile_start"].numpy(), wl.block_m, wl.q.shape[0])
    out = np.full(wl.q.shape, np.nan)
    q = wl.q.double()
    k, v = wl.k.double(), wl.v.double()
    for e in range(len(cu) - 1):
        s0, s1 = int(cu[e]), int(cu[e + 1])
        if s1 == s0 or not covered[s0]:
            continue
        P = int(cc[e + 1] - cc[e])
        kk = torch.cat([torch.tensor(kp[:, cc[e]:cc[e + 1]], dtype=torch.float64),
                        k[s0:s1].transpose(0, 1)], dim=1).repeat_interleave(2, 0)
        vv = torch.cat([torch.tensor(vp[:, cc[e]:cc[e + 1]], dtype=torch.float64),
                        v[s0:s1].transpose(0, 1)], dim=1).repeat_interleave(2, 0)
        L = s1 - s0
        mask = torch.ones(L, P + L, dtype=torch.bool)
        mask[:, P:] = torch.tril(torch.ones(L, L, dtype=torch.bool))
        o = F.scaled_dot_product_attention(q[s0:s1].transpose(0, 1), kk, vv, attn_mask=mask,
                                           scale=128 ** -0.5)
        out[s0:s1] = o.transpose(0, 1).numpy()
    return out


@pytest.mark.parametrize("chunks,dctx", [([(40, 0), (24, 17)], [5, 9]), ([(130, 70)], [])])
def test_prefill_oracle_vs_sdpa64(workloads, chunks, dctx):
    wl = workloads.mixed_workload(dctx, chunks, seed=2, block_m=32, max_len=256)
    cn = cache_np(wl.cache)
    ins = {n: t.numpy() for n, t in wl.inputs.items()}
    kp, vp = okv.dequantize_kv_prefix(cn, ins["cu_cached"], ins["slot_ids"])
    args = (wl.q.float().numpy(), wl.k.float().numpy(), wl.v.float().numpy(), ins["cu_seqlens"],
            ins["tile_start"], wl.block_m, kp, vp, ins["cu_cached"])
    ref = sdpa_prefill64(wl, kp, vp)
    f64 = oat.prefill_attention_f64(*args)
    cov = ~np.isnan(ref[:, 0, 0])
    assert cov.sum() == sum(L for L, _ in chunks)
    assert np.abs(f64[cov] - ref[cov]).max() < 1e-10
    mirror = oat.prefill_attention(*args)
    assert np.isnan(mirror[~cov]).all()
    err = np.abs(mirror[cov] - ref[cov])
    # bf16 P (2^-9 relative) over |v| <= ~4 plus bf16 output rounding
    assert err.max() < 1.5e-2 and err.mean() < 1e-3


@pytest.mark.parametrize("seed", range(6))
def test_work_plan_covers_every_token_once(seed):
    rng = np.random.default_rng(seed)
    B = int(rng.integers(1, 300))
    lens = rng.integers(0, 9000, B)
    nd = int(rng.integers(0, B + 1))
    target = int(rng.choice([41, 128, 256]))
    piece, rows = ows.decode_work_plan(lens, nd, B, target, 64)
    assert piece % 64 == 0 and piece >= 64
    seen = {}
    for b, s, needed in rows:
        if needed == 0:
            continue
        assert b < nd and 0 <= s < needed <= target
        lo, hi = s * piece, min((s + 1) * piece, int(lens[b]) + 1)
        assert lo < hi
        for t in (lo, hi - 1):
            seen.setdefault(b, []).append(t)
        seen.setdefault(("n", b), 0)
        seen[("n", b)] += hi - lo
    for b in range(nd):
        assert seen.get(("n", b), 0) == int(lens[b]) + 1
    assert len(rows) == target + B
    # the build's rule: at least the reference's piece, and the list fits target items whenever
    # nd <= target, with the smallest such piece
    p0 = ows.reference_piece(lens, nd, target, 64)
    assert piece >= p0
    items = sum(1 for r in rows if r[2] > 0)
    if 0 < nd <= target:
        assert items <= target
        if piece > p0:
            n_end = np.asarray(lens[:nd], np.int64) + 1
            assert int(ows.cdiv(n_end, piece - 64).sum()) > target
    else:
        assert piece == p0


def test_work_plan_fits_one_wave_at_config5():
    # 32 sequences of U[128, 4096) tokens: the reference's piece gives 75 pieces per KV head
    # for 64 resident workgroups; the build's piece fits them
    rng = np.random.default_rng(0)
    lens = rng.integers(128, 4096, 32) - 1
    p0 = ows.reference_piece(lens, 32, 64, 128)
    n_end = lens.astype(np.int64) + 1
    assert int(ows.cdiv(n_end, p0).sum()) > 64
    piece, rows = ows.decode_work_plan(lens, 32, 32, 64, 128)
    assert piece > p0 and sum(1 for r in rows if r[2] > 0) <= 64
