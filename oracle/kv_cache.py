"""Oracle for the int8 KV cache writes and reads (test infrastructure only; see oracle/__init__.py).

Restates qwen3-1.7b/kernels.py:
  quantize_kv_prefill      :717-865
  fused_rope_kv_decode     :364-544
  fused_norm_rope_prefill  :547-714 (the same RMSNorm + RoPE, without the cache write)
  dequantize_kv_prefix     :868-970
with the cache container of :11-17 and the allocation of qwen3-1.7b/engine.py:472-492.
All arithmetic is numpy float32 (IEEE round-to-nearest-even, no fused multiply-add), in the
operation order of the reference source.
"""

from dataclasses import dataclass

import numpy as np

from .numerics import F32, bf16_round, butterfly_sum64

EPS_SCALE = F32(1e-6)  # kernels.py:461,475,798,808 `tl.maximum(amax, 1e-6)`
CAL_FLOOR = F32(1e-3)  # kernels.py:765 `tl.full((D,), 1e-3)`
QMAX = F32(127.0)  # kernels.py:461 `/ 127`, clamp at :464


@dataclass
class CacheArrays:
    """numpy twin of `LayerKVCache` (kernels.py:11-17)."""

    k: np.ndarray  # int8 [pool, Hkv, max_len, D]
    v: np.ndarray  # int8 [pool, Hkv, max_len, D]
    k_scale: np.ndarray  # fp32 [pool, Hkv, max_len]
    v_scale: np.ndarray  # fp32 [pool, Hkv, max_len]
    k_calibration: np.ndarray  # fp32 [pool, Hkv, 1, D]

    @staticmethod
    def empty(pool: int, hkv: int, max_len: int, d: int) -> "CacheArrays":
        """Zeroed cache with calibration 1.0, as engine.py:476-492 allocates it."""
        return CacheArrays(
            k=np.zeros((pool, hkv, max_len, d), np.int8),
            v=np.zeros((pool, hkv, max_len, d), np.int8),
            k_scale=np.zeros((pool, hkv, max_len), np.float32),
            v_scale=np.zeros((pool, hkv, max_len), np.float32),
            k_calibration=np.ones((pool, hkv, 1, d), np.float32),
        )

    def copy(self) -> "CacheArrays":
        return CacheArrays(*(a.copy() for a in (self.k, self.v, self.k_scale, self.v_scale,
                                                 self.k_calibration)))


def quantize_rows(x: np.ndarray):
    """Symmetric int8 per row: s = max(max|x|, 1e-6)/127, q = clamp(rint(x/s), -127, 127).

    kernels.py:798-801 (K after calibration), :808-811 (V), :460-469 and :475-478 (decode).
    Returns (q int8 [..., D], s fp32 [...]).
    """
    x = np.asarray(x, dtype=np.float32)
    amax = np.max(np.abs(x), axis=-1)
    s = (np.maximum(amax, EPS_SCALE) / QMAX).astype(np.float32)
    q = np.clip(np.rint((x / s[..., None]).astype(np.float32)), -127.0, 127.0).astype(np.int8)
    return q, s


def calibration(k_chunk: np.ndarray) -> np.ndarray:
    """Per-channel K calibration of a first chunk: max(1e-3, max_t |k[t, d]|) (kernels.py:764-780)."""
    k_chunk = np.asarray(k_chunk, dtype=np.float32)
    if k_chunk.shape[0] == 0:
        return np.full(k_chunk.shape[-1], CAL_FLOOR, np.float32)
    return np.maximum(CAL_FLOOR, np.max(np.abs(k_chunk), axis=0)).astype(np.float32)


def quantize_kv_prefill(k, v, cu_seqlens, slot_ids, cached_lens, num_decoding, cache: CacheArrays):
    """In-place prefill write (kernels.py:717-865).

    k, v: fp32 values of the bf16 inputs, [N, Hkv, D]. Entries b >= num_decoding with a
    non-empty chunk write their tokens at columns [cached_len, cached_len + chunk_len).
    """
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    S = len(cu_seqlens) - 1
    hkv = k.shape[1]
    for b in range(int(num_decoding), S):
        start, end = int(cu_seqlens[b]), int(cu_seqlens[b + 1])
        if end == start:
            continue
        slot, c0 = int(slot_ids[b]), int(cached_lens[b])
        for h in range(hkv):
            kc = k[start:end, h]
            if c0 == 0:
                cache.k_calibration[slot, h, 0] = calibration(kc)
            cal = cache.k_calibration[slot, h, 0]
            kq, ks = quantize_rows((kc / cal[None, :]).astype(np.float32))
            vq, vs = quantize_rows(v[start:end, h])
            cache.k[slot, h, c0:c0 + end - start] = kq
            cache.v[slot, h, c0:c0 + end - start] = vq
            cache.k_scale[slot, h, c0:c0 + end - start] = ks
            cache.v_scale[slot, h, c0:c0 + end - start] = vs


def rmsnorm_rope(x, w, cos, sin, eps):
    """RMSNorm then RoPE of one head row as kernels.py:414-436 computes it, fp32.

    x: [..., D] fp32; w: [D]; cos, sin: [..., D/2] broadcastable. The sum of squares of each
    half uses the fixed wave-butterfly order; rstd = 1/sqrt(mean + eps) with IEEE ops.
    """
    x = np.asarray(x, np.float32)
    d = x.shape[-1]
    h = d // 2
    x1, x2 = x[..., :h], x[..., h:]
    ss = (butterfly_sum64(x1 * x1) + butterfly_sum64(x2 * x2)).astype(np.float32)
    var = (ss / F32(d) + F32(eps)).astype(np.float32)
    rstd = (F32(1.0) / np.sqrt(var)).astype(np.float32)[..., None]
    w = np.asarray(w, np.float32)
    x1 = ((x1 * rstd).astype(np.float32) * w[:h]).astype(np.float32)
    x2 = ((x2 * rstd).astype(np.float32) * w[h:]).astype(np.float32)
    cos = np.asarray(cos, np.float32)
    sin = np.asarray(sin, np.float32)
    o1 = ((x1 * cos).astype(np.float32) - (x2 * sin).astype(np.float32)).astype(np.float32)
    o2 = ((x1 * sin).astype(np.float32) + (x2 * cos).astype(np.float32)).astype(np.float32)
    return o1, o2


def fused_rope_kv_decode(q, k, v, q_norm_weight, k_norm_weight, cos, sin, slot_ids,
                         cache: CacheArrays, cached_lens, num_decoding, eps):
    """Decode-side norm + rope + calibration fold + K/V write (kernels.py:364-544), in place.

    q [B, Hq, D], k/v [B, Hkv, D], cos/sin [B, 1, D/2]: fp32 values of bf16 inputs.
    Returns q_out fp32 (bf16-rounded) [B, Hq, D]; rows b >= num_decoding are NaN (untouched).
    """
    q = np.asarray(q, np.float32)
    B, hq, d = q.shape
    hkv = k.shape[1]
    ratio = hq // hkv
    h = d // 2
    out = np.full(q.shape, np.nan, np.float32)
    for b in range(int(num_decoding)):
        slot = int(slot_ids[b])
        c, s = cos[b, 0], sin[b, 0]
        o1, o2 = rmsnorm_rope(q[b], q_norm_weight, c[None, :], s[None, :], eps)
        cal = cache.k_calibration[slot, :, 0]  # [Hkv, D]
        for hh in range(hq):
            cal_h = cal[hh // ratio]
            out[b, hh, :h] = bf16_round(o1[hh] * cal_h[:h])
            out[b, hh, h:] = bf16_round(o2[hh] * cal_h[h:])
        k1, k2 = rmsnorm_rope(k[b], k_norm_weight, c[None, :], s[None, :], eps)
        col = int(cached_lens[b])
        for j in range(hkv):
            x = np.concatenate([k1[j] / cal[j, :h], k2[j] / cal[j, h:]]).astype(np.float32)
            kq, ks = quantize_rows(x)
            cache.k[slot, j, col] = kq
            cache.k_scale[slot, j, col] = ks
            vq, vs = quantize_rows(np.asarray(v[b, j], np.float32))
            cache.v[slot, j, col] = vq
            cache.v_scale[slot, j, col] = vs
    return out


def fused_norm_rope_prefill(q, k, q_norm_weight, k_norm_weight, cos, sin, eps):
    """Prefill q/k RMSNorm + RoPE over packed tokens (kernels.py:547-662, wrapper :665-714).

    q [N, Hq, D], k [N, Hkv, D], cos/sin [N, 1, D/2]: fp32 values of bf16 inputs; one cos/sin row
    per token for all of its heads (:627-634). Returns (q_out, k_out) fp32 (bf16-rounded, the
    bf16 store of :636-662).
    """
    q1, q2 = rmsnorm_rope(q, q_norm_weight, cos, sin, eps)
    k1, k2 = rmsnorm_rope(k, k_norm_weight, cos, sin, eps)
    return (bf16_round(np.concatenate([q1, q2], axis=-1)),
            bf16_round(np.concatenate([k1, k2], axis=-1)))


def dequantize_kv_prefix(cache: CacheArrays, cu_cached, slot_ids):
    """int8 prefix -> bf16 rows (kernels.py:868-932): k = bf16((q*ks)*cal), v = bf16(q*vs).

    Returns (k_out, v_out) fp32 (bf16-rounded) [Hkv, total, D].
    """
    hkv, d = cache.k.shape[1], cache.k.shape[3]
    total = int(cu_cached[-1])
    k_out = np.zeros((hkv, total, d), np.float32)
    v_out = np.zeros((hkv, total, d), np.float32)
    for b in range(len(cu_cached) - 1):
        s0, n = int(cu_cached[b]), int(cu_cached[b + 1]) - int(cu_cached[b])
        if n <= 0:
            continue
        slot = int(slot_ids[b])
        for h in range(hkv):
            kq = cache.k[slot, h, :n].astype(np.float32)
            ks = cache.k_scale[slot, h, :n][:, None]
            cal = cache.k_calibration[slot, h, 0][None, :]
            k_out[h, s0:s0 + n] = bf16_round(((kq * ks).astype(np.float32) * cal).astype(np.float32))
            vq = cache.v[slot, h, :n].astype(np.float32)
            vs = cache.v_scale[slot, h, :n][:, None]
            v_out[h, s0:s0 + n] = bf16_round((vq * vs).astype(np.float32))
    return k_out, v_out
