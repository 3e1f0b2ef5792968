"""Attention oracle (test infrastructure only; see oracle/__init__.py).

decode_attention      qwen3-1.7b/kernels.py:84-213 (split kernel), :216-264 (combine),
                      :272-361 (wrapper): scores = dot(q, k_int8) * (k_scale * scale), softmax
                      with exp, P rounded as bf16(p * v_scale) before PV (kernels.py:186).
decode_attention_split the same computed split by split with the log-sum-exp merge of :255-259.
prefill_attention     qwen3-1.7b/kernels.py:987-1126: per tile row, prefix keys then chunk keys
                      n <= m, scores * (D^-0.5 * log2 e), exp2, P rounded to bf16 before PV
                      (:1068, :1113), out = acc / l or 0 when l == 0 (:1118).
*_f64                 textbook float64 forms with no intermediate rounding.
"""

import numpy as np

from .numerics import F32, bf16_round

LOG2E = 1.4426950408889634


def _decode_rows(cache, slot, hk, n):
    k = cache.k[slot, hk, :n].astype(np.float32)
    v = cache.v[slot, hk, :n].astype(np.float32)
    return k, v, cache.k_scale[slot, hk, :n], cache.v_scale[slot, hk, :n]


def _partial(q_row, k, v, ks, vs, scale):
    """One program's online-softmax state over a token range, single pass (kernels.py:153-189)."""
    s = ((k @ q_row).astype(np.float32) * (ks * F32(scale)).astype(np.float32)).astype(np.float32)
    m = np.max(s)
    p = np.exp((s - m).astype(np.float32)).astype(np.float32)
    l = np.sum(p, dtype=np.float32)
    pv = bf16_round((p * vs).astype(np.float32))
    acc = (pv @ v).astype(np.float32)
    return m, l, acc


def decode_attention(q, cache, cached_lens, slot_ids, num_decoding, scale, splits=None):
    """Reference-rounding decode attention. q: fp32 values of bf16 [B, Hq, D].

    `splits`: optional list giving each sequence's token pieces [(start, end), ...]; the partials
    are merged as the combine kernel does. None = one piece per sequence.
    Returns fp32 (bf16-rounded) [B, Hq, D]; rows >= num_decoding are NaN.
    """
    q = np.asarray(q, np.float32)
    B, hq, d = q.shape
    hkv = cache.k.shape[1]
    ratio = hq // hkv
    out = np.full(q.shape, np.nan, np.float32)
    for b in range(int(num_decoding)):
        slot, n = int(slot_ids[b]), int(cached_lens[b]) + 1
        pieces = [(0, n)] if splits is None else splits[b]
        for hk in range(hkv):
            k, v, ks, vs = _decode_rows(cache, slot, hk, n)
            for g in range(ratio):
                h = hk * ratio + g
                parts = [_partial(q[b, h], k[a:e], v[a:e], ks[a:e], vs[a:e], scale)
                         for a, e in pieces]
                if len(parts) == 1:
                    m, l, acc = parts[0]
                    out[b, h] = bf16_round(acc / l)
                else:  # kernels.py:255-259
                    mx = max(p[0] for p in parts)
                    w = [np.exp(F32(p[0] - mx)) for p in parts]
                    num = sum(p[2] * wi for p, wi in zip(parts, w))
                    den = sum(p[1] * wi for p, wi in zip(parts, w))
                    out[b, h] = bf16_round((num / den).astype(np.float32))
    return out


def decode_attention_f64(q, cache, cached_lens, slot_ids, num_decoding, scale):
    """Textbook float64 softmax attention over the dequantized cache (no intermediate rounding)."""
    q = np.asarray(q, np.float64)
    B, hq, d = q.shape
    hkv = cache.k.shape[1]
    ratio = hq // hkv
    out = np.full(q.shape, np.nan, np.float64)
    for b in range(int(num_decoding)):
        slot, n = int(slot_ids[b]), int(cached_lens[b]) + 1
        for hk in range(hkv):
            kd = cache.k[slot, hk, :n].astype(np.float64) * cache.k_scale[slot, hk, :n, None]
            vd = cache.v[slot, hk, :n].astype(np.float64) * cache.v_scale[slot, hk, :n, None]
            for g in range(ratio):
                h = hk * ratio + g
                s = kd @ q[b, h] * scale
                p = np.exp(s - s.max())
                out[b, h] = (p @ vd) / p.sum()
    return out


def prefill_rows(cu_seqlens, tile_start, block_m, n_tokens):
    """Packed rows the tiles of `tile_start` cover (each tile stays inside one entry, E:318-327)."""
    covered = np.zeros(n_tokens, bool)
    cu = np.asarray(cu_seqlens)
    for r0 in np.asarray(tile_start):
        r0 = int(r0)
        if r0 < 0:
            continue
        e = int(np.searchsorted(cu, r0, side="right") - 1)
        covered[r0:min(r0 + block_m, int(cu[e + 1]))] = True
    return covered


def prefill_attention(q, k, v, cu_seqlens, tile_start, block_m, k_prefix, v_prefix, cu_cached,
                      rows=None):
    """Reference-rounding chunked-prefill attention.

    q [N, Hq, D], k/v [N, Hkv, D]: fp32 values of bf16 inputs; k_prefix/v_prefix
    [Hkv, total_cached, D] bf16-rounded (from dequantize_kv_prefix). Returns fp32
    (bf16-rounded) [N, Hq, D]; rows no tile covers are NaN. `rows`: compute only these packed
    rows (the others stay NaN), for long prefills checked on a sample.
    """
    q = np.asarray(q, np.float32)
    N, hq, d = q.shape
    hkv = k.shape[1]
    ratio = hq // hkv
    qk_scale = F32(d ** -0.5 * LOG2E)
    out = np.full(q.shape, np.nan, np.float32)
    covered = prefill_rows(cu_seqlens, tile_start, block_m, N)
    if rows is not None:
        keep = np.zeros(N, bool)
        keep[np.asarray(rows)] = True
        covered &= keep
    cu = np.asarray(cu_seqlens)
    for m in np.nonzero(covered)[0]:
        e = int(np.searchsorted(cu, m, side="right") - 1)
        s0 = int(cu[e])
        p0, p1 = int(cu_cached[e]), int(cu_cached[e + 1])
        for h in range(hq):
            hk = h // ratio
            kk = np.concatenate([k_prefix[hk, p0:p1], k[s0:m + 1, hk]]).astype(np.float32)
            vv = np.concatenate([v_prefix[hk, p0:p1], v[s0:m + 1, hk]]).astype(np.float32)
            s = ((kk @ q[m, h]).astype(np.float32) * qk_scale).astype(np.float32)
            p = np.exp2((s - s.max()).astype(np.float32)).astype(np.float32)
            l = np.sum(p, dtype=np.float32)
            acc = (bf16_round(p) @ vv).astype(np.float32)
            out[m, h] = bf16_round(acc / l)
    return out


def prefill_attention_f64(q, k, v, cu_seqlens, tile_start, block_m, k_prefix, v_prefix, cu_cached):
    """Textbook float64 causal attention over [prefix || chunk]; same row coverage."""
    q = np.asarray(q, np.float64)
    N, hq, d = q.shape
    hkv = k.shape[1]
    ratio = hq // hkv
    out = np.full(q.shape, np.nan, np.float64)
    covered = prefill_rows(cu_seqlens, tile_start, block_m, N)
    cu = np.asarray(cu_seqlens)
    for m in np.nonzero(covered)[0]:
        e = int(np.searchsorted(cu, m, side="right") - 1)
        s0 = int(cu[e])
        p0, p1 = int(cu_cached[e]), int(cu_cached[e + 1])
        for h in range(hq):
            hk = h // ratio
            kk = np.concatenate([k_prefix[hk, p0:p1], k[s0:m + 1, hk]]).astype(np.float64)
            vv = np.concatenate([v_prefix[hk, p0:p1], v[s0:m + 1, hk]]).astype(np.float64)
            s = kk @ q[m, h] * d ** -0.5
            p = np.exp(s - s.max())
            out[m, h] = (p @ vv) / p.sum()
    return out
