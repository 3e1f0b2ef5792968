"""Prefill attention on peaked scores and off-scale V.

The prefill kernel keeps a lazy running max per row: it moves only when a score exceeds it by
more than 8 log2 units, and only then rescales the row sums and the accumulators (softmax_rescale
in prefill_attention.hip; the reference rescales at every new maximum, kernels.py:1060-1066,
1105-1111). With N(0, 1) inputs a row's maximum never climbs that far after a piece's first
tile, so these tests build inputs where it must:

* ramp: every key of a row's 64-key tile t carries lam_t * u (u = +-1 per KV head, lam_t =
  step * (t + 1), prefix tiles then chunk tiles), and every query row is u plus a part orthogonal
  to u, so each tile's scores sit step * 128 * D^-0.5 * log2(e) (16.3 per unit step) above the
  previous tile's: the max moves at every tile boundary of every piece;
* planted: near-flat scores plus one key per work piece (from the device's own work list,
  ie_prefill_attention_plan) in a non-first tile of the piece: in the prefix 11.2 log2 units
  above the rest, so the jump moves the max while the keys before it still carry a share of the
  softmax mass that a wrong rescale factor would misweigh; in the chunk 11.2 more per chunk
  tile (sub-blocks of one entry cut their chunk tiles into pieces at different places, so a key
  planted for one sub-block can sit in another's first tile, and a later key must still jump);
* a config-4 mixed step through the attention layer with q/k norm weights times 4 (scores of
  standard deviation ~23 log2 units).

Prefix K is quantized with power-of-two scales and calibration 1, so bf16(k_int8 * k_scale * cal)
(the reference's dequantization) and the kernel's folded form k_int8 * (k_scale * qk_scale) are
exact and both sides see the same scores; large scores then do not amplify rounding differences
between the two. Each test shows from float64 scores that its construction drives the branch
(the kernel moves at least whenever the exact running max over a piece's tiles jumps by more than
8, since its lazy max never exceeds the exact one), then checks the outputs against the oracle
with the north star's bf16 tolerance, absolute and scale-normalised. V is scaled by 1e-3 and 1e2
as well as 1.
"""

import importlib

import numpy as np
import pytest
import torch

from helpers import (PLAN_FIELDS, assert_attn_close, assert_cache_bitwise, bf16_np, cache_np,
                     prefill_plan, say)
from oracle import attention as oat
from oracle import kv_cache as okv

pytestmark = pytest.mark.gpu
HQ, HKV, D = 16, 8, 128
QK = D ** -0.5 * 1.4426950408889634  # log2 units per unit of q . k
SLACK = 8.0  # the kernel's lazy-max slack, log2 units
F = {n: i for i, n in enumerate(PLAN_FIELDS)}


def pow2_quantize(kf):
    """int8 rows with a power-of-two scale each (the largest that keeps |q| <= 127), so that
    q * scale, and (q * scale) * 1.0 rounded to bf16, are exact."""
    amax = np.maximum(np.abs(kf).max(-1), 1e-30)
    e = np.clip(np.floor(np.log2(127.0 / amax)), -100, 100)
    q = np.clip(np.rint(kf * 2.0 ** e[..., None]), -127, 127).astype(np.int8)
    return q, (2.0 ** -e).astype(np.float32)


def _u_and_q(rng, L):
    """u (+-1 per KV head) and L query rows per head: u of the head's KV head plus a N(0, 1)
    part orthogonal to it (q . u = 128 before bf16 rounding)."""
    u = rng.choice([-1.0, 1.0], size=(HKV, D))
    uq = np.repeat(u, HQ // HKV, axis=0)
    z = rng.standard_normal((L, HQ, D))
    z -= (z * uq).sum(-1, keepdims=True) / D * uq
    return u, uq + z


def _set_prefix(cache, slot, kf, vf):
    kq, ks = pow2_quantize(kf)
    vq, vs = okv.quantize_rows(vf.astype(np.float32))
    P = kf.shape[1]
    cache.k[slot, :, :P] = torch.from_numpy(kq)
    cache.k_scale[slot, :, :P] = torch.from_numpy(ks)
    cache.v[slot, :, :P] = torch.from_numpy(vq)
    cache.v_scale[slot, :, :P] = torch.from_numpy(vs)
    cache.k_calibration[slot] = 1.0


def ramp_workload(workloads, chunks, seed, step=1.0, knoise=1.0, v_mult=1.0, block_m=128):
    max_len = -(-max(L + c for L, c in chunks) // 64) * 64
    wl = workloads.mixed_workload([], chunks, seed=seed, block_m=block_m, max_len=max_len)
    rng = np.random.default_rng(seed + 1000)
    cu = wl.inputs["cu_seqlens"].numpy()
    q, k, v = (t.float().numpy().copy() for t in (wl.q, wl.k, wl.v))
    for e, (L, P) in enumerate(chunks):
        s0 = int(cu[e])
        u, q[s0:s0 + L] = _u_and_q(rng, L)
        lam_p = step * (np.arange(P) // 64 + 1)
        kf = knoise * rng.standard_normal((HKV, P, D)) + lam_p[None, :, None] * u[:, None, :]
        _set_prefix(wl.cache, e, kf, rng.standard_normal((HKV, P, D)) * v_mult)
        lam_c = step * (-(-P // 64) + np.arange(L) // 64 + 1)
        k[s0:s0 + L] = knoise * rng.standard_normal((L, HKV, D)) + lam_c[:, None, None] * u[None]
        v[s0:s0 + L] = rng.standard_normal((L, HKV, D)) * v_mult
    for t, x in ((wl.q, q), (wl.k, k), (wl.v, v)):
        t.copy_(torch.from_numpy(x).bfloat16())
    return wl


def planted_workload(workloads, native, dev, chunks, seed, v_mult=1.0, block_m=128):
    """Near-flat scores (keys 0.1 N(0, 1)) and, for every piece of two or more tiles in the
    device's work list, one key at a random position of a random non-first tile of the piece:
    u * 11/16 (11.2 log2 units) in the prefix, u * 11/16 * (2 + chunk tile) in the chunk, at a
    position of the tile that at least half the sub-block's rows see."""
    max_len = -(-max(L + c for L, c in chunks) // 64) * 64
    wl = workloads.mixed_workload([], chunks, seed=seed, block_m=block_m, max_len=max_len)
    rng = np.random.default_rng(seed + 2000)
    cu = wl.inputs["cu_seqlens"].numpy()
    q, k, v = (t.float().numpy().copy() for t in (wl.q, wl.k, wl.v))
    us, kpre = [], []
    for e, (L, P) in enumerate(chunks):
        s0 = int(cu[e])
        u, q[s0:s0 + L] = _u_and_q(rng, L)
        us.append(u)
        kpre.append(0.1 * rng.standard_normal((HKV, P, D)))
        k[s0:s0 + L] = 0.1 * rng.standard_normal((L, HKV, D))
        v[s0:s0 + L] = rng.standard_normal((L, HKV, D)) * v_mult
    for t, x in ((wl.q, q), (wl.k, k)):
        t.copy_(torch.from_numpy(x).bfloat16())
    plan = prefill_plan(native, workloads.mixed_to(wl, dev))
    entry_of = {int(s): e for e, s in enumerate(cu[:-1])}
    planted = 0
    for r in plan[plan[:, F["found"]] == 1]:
        kb, ke = int(r[F["kt_begin"]]), int(r[F["kt_end"]])
        if ke - kb < 2 or r[F["hk"]] != 0:  # every KV head runs the same pieces
            continue
        e = entry_of[int(r[F["seq_start"]])]
        npt, P, s0 = int(r[F["npt"]]), int(r[F["P"]]), int(r[F["seq_start"]])
        t = int(rng.integers(kb + 1, ke))
        if t < npt:  # a prefix key
            pos = 64 * t + int(rng.integers(0, min(64, P - 64 * t)))
            kpre[e][:, pos] = us[e] * (11 / 16)
        else:  # a chunk key, visible to the sub-block's rows at or after it
            n_vis = int(r[F["r1"]]) - s0
            pos = 64 * (t - npt) + int(rng.integers(0, min(8, n_vis - 64 * (t - npt))))
            k[s0 + pos] = us[e] * (11 / 16) * (2 + t - npt)
        planted += 1
    for e, (L, P) in enumerate(chunks):
        _set_prefix(wl.cache, e, kpre[e], rng.standard_normal((HKV, P, D)) * v_mult)
    wl.k.copy_(torch.from_numpy(k).bfloat16())
    wl.v.copy_(torch.from_numpy(v).bfloat16())
    assert planted > 0
    return wl


def tile_maxima(q, k, cache, ins, r0, r1, s0, e, hk):
    """float64 scores (log2 units) of rows [r0, r1) of entry e for the two query heads of KV head
    hk, reduced to the max of each 64-key tile in the kernel's tile order (prefix tiles, then
    chunk tiles; -inf where a row sees no key of the tile). Returns [r1 - r0, 2, tiles]."""
    slot = int(ins["slot_ids"][e])
    P = int(ins["cu_cached"][e + 1] - ins["cu_cached"][e])
    kp = (cache.k[slot, hk, :P].astype(np.float64) * cache.k_scale[slot, hk, :P, None] *
          cache.k_calibration[slot, hk, 0][None, :])
    nvis = r1 - s0
    kc = k[s0:r1, hk].astype(np.float64)
    out = []
    for h in (2 * hk, 2 * hk + 1):
        qq = q[r0:r1, h].astype(np.float64)
        sp = qq @ kp.T * QK
        sc = qq @ kc.T * QK
        rows = np.arange(r0, r1)[:, None] - s0
        sc = np.where(np.arange(nvis)[None, :] <= rows, sc, -np.inf)
        npt, nct = -(-P // 64), -(-nvis // 64)
        sp = np.pad(sp, ((0, 0), (0, 64 * npt - P)), constant_values=-np.inf)
        sc = np.pad(sc, ((0, 0), (0, 64 * nct - nvis)), constant_values=-np.inf)
        out.append(np.concatenate([sp.reshape(len(qq), npt, 64).max(-1),
                                   sc.reshape(len(qq), nct, 64).max(-1)], axis=1))
    return np.stack(out, axis=1)


def rescale_coverage(plan, q, k, cache, ins):
    """For every piece of two or more tiles in the work list: the fraction of its (row, query
    head) pairs that see a key after the piece's first tile and whose exact running max over the
    piece's tiles jumps by more than SLACK there (so the kernel's rescale branch runs for them).
    Returns (per-piece fractions, number of such (row, head) pairs, pieces by form)."""
    cu = ins["cu_seqlens"]
    entry_of = {int(s): e for e, s in enumerate(cu[:-1])}
    cache_tm = {}
    fracs, moved_total, forms = [], 0, {"prefix": 0, "chunk": 0, "straddle": 0, "unsplit": 0}
    for r in plan[plan[:, F["found"]] == 1]:
        kb, ke = int(r[F["kt_begin"]]), int(r[F["kt_end"]])
        if ke - kb < 2:
            continue
        key = (int(r[F["sb"]]), int(r[F["hk"]]))
        if key not in cache_tm:
            s0 = int(r[F["seq_start"]])
            cache_tm[key] = tile_maxima(q, k, cache, ins, int(r[F["r0"]]), int(r[F["r1"]]), s0,
                                        entry_of[s0], key[1])
        tm = cache_tm[key][:, :, kb:ke]
        run = np.maximum.accumulate(tm, axis=-1)
        jump = tm[..., 1:] > run[..., :-1] + SLACK
        sees = np.isfinite(tm[..., 1:]).any(-1)
        moved = jump.any(-1)
        npt = int(r[F["npt"]])
        form = ("unsplit" if r[F["npieces"]] == 1 else "straddle" if kb < npt < ke
                else "prefix" if ke <= npt else "chunk")
        forms[form] += 1
        if sees.any():
            fracs.append(moved[sees].mean())
            moved_total += int(moved.sum())
    return np.array(fracs), moved_total, forms


def oracle_prefill(wl):
    ins = {n: t.cpu().numpy() for n, t in wl.inputs.items()}
    kp, vp = okv.dequantize_kv_prefix(cache_np(wl.cache), ins["cu_cached"], ins["slot_ids"])
    return oat.prefill_attention(bf16_np(wl.q), bf16_np(wl.k), bf16_np(wl.v), ins["cu_seqlens"],
                                 ins["tile_start"], wl.block_m, kp, vp, ins["cu_cached"])


def run_and_check(ie, workloads, native, dev, wl, what, min_frac, v_mult, forms_needed=(),
                  min_pieces_moving=1.0):
    """Coverage first: in every piece of two or more tiles, at least min_frac of the (row, head)
    pairs that see its later tiles take the rescale branch, and at least min_pieces_moving of
    those pieces have one that does; then the outputs against the oracle."""
    g = workloads.mixed_to(wl, dev)
    plan = prefill_plan(native, g)
    ins = {n: t.numpy() for n, t in wl.inputs.items()}
    fr, moved, forms = rescale_coverage(plan, bf16_np(wl.q), bf16_np(wl.k), cache_np(wl.cache),
                                        ins)
    say(f"{what}: pieces {forms}; rescale branch for {moved} (row, head) pairs, per-piece "
        f"fraction min {fr.min():.3f} mean {fr.mean():.3f}, pieces with a move "
        f"{np.mean(fr > 0):.3f}")
    for f in forms_needed:
        assert forms[f] > 0, f"{what}: the work list has no {f} piece"
    assert len(fr) > 0 and np.mean(fr > 0) >= min_pieces_moving, \
        f"{what}: pieces without the branch"
    assert np.mean(fr[fr > 0] >= min_frac) >= min_pieces_moving, \
        f"{what}: construction misses the branch"
    ref = oracle_prefill(wl)
    gi = g.inputs
    out = ie.prefill_attention(g.q, g.k, g.v, gi["seq_ids"], gi["cu_seqlens"], gi["tile_start"],
                               g.cache, gi["slot_ids"], gi["cu_cached"], g.block_m)
    torch.cuda.synchronize()
    cov = ~np.isnan(ref[:, 0, 0])
    assert_attn_close(bf16_np(out)[cov], ref[cov], what,
                      abs_scale=max(1.0, v_mult) * max(1.0, float(np.abs(ref[cov]).max())))


@pytest.mark.parametrize("v_mult", [1.0, 1e-3, 1e2])
@pytest.mark.parametrize("chunks,forms", [
    ([(512, 1536)], ("prefix", "chunk")),       # split prefix pieces and chunk pieces
    ([(512, 0), (512, 1536)], ("prefix", "chunk")),  # config 4's chunks
    ([(64, 1000 + 250 * i) for i in range(16)], ("straddle",)),
    ([(700, 0)], ("unsplit",)),                 # a chunk alone: unsplit causal pieces
])
def test_prefill_ramp_moves_every_tile(ie, workloads, native, dev, chunks, forms, v_mult):
    """Every piece takes the branch, for at least 95 % of the (row, head) pairs that see its
    later tiles (a row that sees only the first few keys of a causal diagonal tile can fall
    short of the jump; the mean is above 99 %)."""
    say(f"prefill ramp {len(chunks)} chunks {chunks[:2]}..., v x {v_mult}")
    wl = ramp_workload(workloads, chunks, seed=41, v_mult=v_mult)
    run_and_check(ie, workloads, native, dev, wl, f"ramp {chunks[:2]} v x {v_mult}", 0.95,
                  v_mult, forms)


@pytest.mark.parametrize("v_mult", [1.0, 1e-3, 1e2])
@pytest.mark.parametrize("chunks", [
    [(512, 1536)], [(64, 1000 + 250 * i) for i in range(16)], [(300, 5000), (64, 9000)],
])
def test_prefill_planted_key_per_piece(ie, workloads, native, dev, chunks, v_mult):
    """Every piece takes the branch, for at least a quarter of the (row, head) pairs that see
    its later tiles (all of them in prefix pieces; rows before a planted chunk key do not see
    it)."""
    say(f"prefill planted {len(chunks)} chunks {chunks[:2]}..., v x {v_mult}")
    wl = planted_workload(workloads, native, dev, chunks, seed=43, v_mult=v_mult)
    run_and_check(ie, workloads, native, dev, wl, f"planted {chunks[:2]} v x {v_mult}", 0.25,
                  v_mult)


@pytest.mark.parametrize("v_mult", [1.0, 1e2])
def test_mixed_step_peaked_config4(ie, workloads, native, dev, v_mult):
    """Config 4 through the attention layer (prefill norm/RoPE, KV write, prefill attention,
    fused decode) with q/k norm weights x 4: every prefill and decode row against the oracle and
    the cache bit for bit. Chunk B's 1536 cached tokens hold power-of-two-scaled K (calibration
    1); V (raw rows and every cached row) is scaled by v_mult."""
    ms = importlib.import_module("test_mixed_step_gpu")
    wl = workloads.config4(seed=12)
    nd = len(wl.decode_ctx)
    rng = np.random.default_rng(12)
    slot_b = nd + 1
    _set_prefix(wl.cache, slot_b, 4.0 * rng.standard_normal((HKV, 1536, D)),
                rng.standard_normal((HKV, 1536, D)))
    wl.cache.v_scale.mul_(v_mult)
    al, g, qkv, q, k, v, qw, kw, cos, sin = ms.step_setup(workloads, wl, dev, seed=13)
    qw.mul_(4.0)
    kw.mul_(4.0)
    v.mul_(v_mult)
    ins = {n: t.cpu().numpy() for n, t in g.inputs.items()}
    # the step's post-norm q and k, for the coverage check
    q_p, k_p = okv.fused_norm_rope_prefill(bf16_np(q), bf16_np(k), bf16_np(qw), bf16_np(kw),
                                           bf16_np(cos), bf16_np(sin), ms.EPS)
    ref, ref_cache = ms.oracle_step(q, k, v, qw, kw, cos, sin, g.cache, ins, wl.block_m)
    plan = prefill_plan(native, g)
    fr, moved, forms = rescale_coverage(plan, q_p, k_p, ref_cache, ins)
    say(f"peaked config 4 v x {v_mult}: pieces {forms}; rescale branch for {moved} (row, head) "
        f"pairs; pieces with a move {np.mean(fr > 0):.2f}")
    assert np.mean(fr > 0) >= 0.5 and moved > 1000, "construction misses the branch"
    out = ms.run_step(al, g, q, k, v, qw, kw, cos, sin)
    torch.cuda.synchronize()
    o = bf16_np(out)
    rows = ~np.isnan(ref[:, 0, 0])
    # peaked outputs are single V rows (magnitude up to ~4): one bf16 step is 2^-6 there
    sc = max(1.0, v_mult) * max(1.0, float(np.abs(ref[rows]).max()))
    assert_attn_close(o[:nd], ref[:nd], f"peaked config 4 v x {v_mult}: decode rows",
                      abs_scale=sc)
    assert_attn_close(o[rows], ref[rows], f"peaked config 4 v x {v_mult}: all rows",
                      abs_scale=sc)
    assert_cache_bitwise(g.cache, ref_cache, "peaked config 4 cache")
