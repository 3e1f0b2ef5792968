"""Pins the oracle's int8 quantize / calibration / decode-write / dequantize arithmetic against
known answers and float64 library math (CPU only)."""

import numpy as np
import pytest
import torch

from oracle import kv_cache as okv
from oracle.numerics import bf16_round, butterfly_sum64

F32 = np.float32


def test_zero_row_uses_scale_floor():
    q, s = okv.quantize_rows(np.zeros((3, 128), np.float32))
    assert np.all(q == 0)
    assert np.all(s == F32(1e-6) / F32(127))


@pytest.mark.parametrize("a", [0.37, 5.0, 1e-3, 3.0e4])
@pytest.mark.parametrize("idx", [0, 63, 127])
def test_one_hot_maps_to_127(a, idx):
    for sign in (1, -1):
        x = np.zeros(128, np.float32)
        x[idx] = sign * a
        q, s = okv.quantize_rows(x)
        assert s == F32(a) / F32(127)
        assert q[idx] == sign * 127 and np.count_nonzero(q) == 1


def test_exact_ties_round_half_to_even():
    # max |x| = 127 gives s == 1 exactly, so x/s == x and the .5 ties are exact.
    x = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, 126.5, -126.5] + [0.0] * 118,
                 np.float32)
    q, s = okv.quantize_rows(x)
    assert s == F32(1.0)
    assert q[:10].tolist() == [127, 0, 2, 2, 0, -2, -2, 4, 126, -126]


def test_amax_element_is_always_127_and_roundtrip_bound():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((4096, 128)) * rng.uniform(1e-3, 50, (4096, 1))).astype(np.float32)
    q, s = okv.quantize_rows(x)
    assert np.all(np.abs(q).max(axis=1) == 127)
    err = np.abs(x - q.astype(np.float64) * s[:, None].astype(np.float64))
    assert np.all(err <= s[:, None] * (0.5 + 1e-6))


def test_calibration_floor_and_channel_max():
    k = np.zeros((5, 128), np.float32)
    k[2, 7] = -3.0
    k[4, 9] = 0.5e-3
    cal = okv.calibration(k)
    assert cal[7] == F32(3.0)
    assert cal[9] == F32(1e-3)  # below the floor
    assert np.all(np.delete(cal, [7]) == F32(1e-3))


def _int_rows(rng, n):
    """Integer rows in [-127, 127] with |max| == 127 in every row."""
    r = rng.integers(-126, 127, size=(n, 128)).astype(np.float32)
    r[np.arange(n), rng.integers(0, 128, n)] = 127 * rng.choice([-1, 1], n)
    return r


def test_prefill_write_known_answer_with_stored_calibration():
    """cached_len > 0: the stored calibration (powers of two) is used, not recomputed.
    k = cal * r with integer rows r (max |r| = 127) quantizes to exactly r with scale 1."""
    rng = np.random.default_rng(1)
    pool, hkv, L = 4, 2, 64
    cache = okv.CacheArrays.empty(pool, hkv, L, 128)
    cal = (2.0 ** rng.integers(-3, 4, size=(hkv, 128))).astype(np.float32)
    cache.k_calibration[2, :, 0] = cal
    n, c0 = 9, 5
    r_k = np.stack([_int_rows(rng, n) for _ in range(hkv)], axis=1)  # [n, hkv, D]
    r_v = np.stack([_int_rows(rng, n) for _ in range(hkv)], axis=1)
    k = r_k * cal[None]
    v = r_v.copy()
    cu = np.array([0, 1, 1 + n])  # entry 0 decoding (skipped), entry 1 prefilling
    okv.quantize_kv_prefill(np.concatenate([np.zeros((1, hkv, 128), np.float32), k]),
                            np.concatenate([np.zeros((1, hkv, 128), np.float32), v]),
                            cu, np.array([0, 2]), np.array([0, c0]), 1, cache)
    assert np.array_equal(cache.k_calibration[2, :, 0], cal)
    assert np.array_equal(cache.k[2, :, c0:c0 + n], r_k.transpose(1, 0, 2).astype(np.int8))
    assert np.array_equal(cache.v[2, :, c0:c0 + n], r_v.transpose(1, 0, 2).astype(np.int8))
    assert np.all(cache.k_scale[2, :, c0:c0 + n] == 1.0)
    assert np.all(cache.v_scale[2, :, c0:c0 + n] == 1.0)
    # nothing else written: the decoding entry's slot and columns outside the chunk
    assert not cache.k[0].any() and not cache.k[2, :, :c0].any() and not cache.k[2, :, c0 + n:].any()


def test_prefill_first_chunk_calibration_known_answer():
    """cached_len == 0: cal[d] = max(1e-3, max_t |k[t,d]|) is recomputed and stored."""
    hkv, n = 1, 6
    cache = okv.CacheArrays.empty(2, hkv, 16, 128)
    cache.k_calibration[:] = 7.0  # stale value that must be overwritten
    k = np.zeros((n, hkv, 128), np.float32)
    expect = np.full(128, 1e-3, np.float32)
    for d in range(0, 128, 3):
        m = F32(2.0 ** ((d % 7) - 3))
        k[d % n, 0, d] = -m
        expect[d] = m
    okv.quantize_kv_prefill(k, k, np.array([0, n]), np.array([1]), np.array([0]), 0, cache)
    assert np.array_equal(cache.k_calibration[1, 0, 0], expect)
    # channel maxima become exactly +-127 in their token's row (x / cal = +-1 is that row's max)
    for d in range(0, 128, 3):
        assert cache.k[1, 0, d % n, d] == -127


def test_decode_write_matches_float64_norm_rope():
    rng = np.random.default_rng(2)
    B, hq, hkv = 3, 16, 8
    gen = torch.Generator().manual_seed(0)
    q = torch.randn(B, hq, 128, generator=gen).bfloat16().float().numpy()
    k = torch.randn(B, hkv, 128, generator=gen).bfloat16().float().numpy()
    v = torch.randn(B, hkv, 128, generator=gen).bfloat16().float().numpy()
    qw = (1 + 0.1 * torch.randn(128, generator=gen)).bfloat16().float().numpy()
    kw = (1 + 0.1 * torch.randn(128, generator=gen)).bfloat16().float().numpy()
    ang = rng.uniform(0, 100, (B, 1, 64))
    cos = torch.tensor(np.cos(ang)).bfloat16().float().numpy()
    sin = torch.tensor(np.sin(ang)).bfloat16().float().numpy()
    cache = okv.CacheArrays.empty(5, hkv, 32, 128)
    cache.k_calibration[:] = rng.uniform(0.5, 3, cache.k_calibration.shape).astype(np.float32)
    slots, lens = np.array([4, 0, 2]), np.array([7, 0, 31])
    qo = okv.fused_rope_kv_decode(q, k, v, qw, kw, cos, sin, slots, cache, lens, 2, 1e-6)
    assert np.isnan(qo[2]).all()  # b >= num_decoding untouched
    assert not cache.k[2].any()

    # float64 textbook: torch RMSNorm then RoPE as a complex rotation
    def norm_rope64(x, w, c, s):
        xn = torch.nn.functional.rms_norm(torch.tensor(x, dtype=torch.float64), (128,),
                                          torch.tensor(w, dtype=torch.float64), eps=1e-6).numpy()
        z = (xn[..., :64] + 1j * xn[..., 64:]) * (c + 1j * s)
        return np.concatenate([z.real, z.imag], axis=-1)

    for b in range(2):
        slot = slots[b]
        cal = cache.k_calibration[slot, :, 0].astype(np.float64)
        ref_q = norm_rope64(q[b], qw, cos[b, 0], sin[b, 0]) * np.repeat(cal, 2, axis=0)
        assert np.allclose(qo[b], ref_q, rtol=2 ** -8, atol=1e-6)
        ref_k = norm_rope64(k[b], kw, cos[b, 0], sin[b, 0]) / cal
        ks64 = np.abs(ref_k).max(axis=1) / 127
        assert np.allclose(cache.k_scale[slot, :, lens[b]], ks64, rtol=1e-5)
        kq64 = np.rint(ref_k / ks64[:, None])
        diff = np.abs(cache.k[slot, :, lens[b]].astype(np.int64) - kq64)
        assert diff.max() <= 1 and np.mean(diff) < 0.01
        vs64 = np.abs(v[b].astype(np.float64)).max(axis=1) / 127
        assert np.allclose(cache.v_scale[slot, :, lens[b]], vs64, rtol=1e-6)
        assert np.abs(cache.v[slot, :, lens[b]] - np.rint(v[b] / vs64[:, None])).max() <= 1


def _norm_rope64(x, w, c, s):
    """float64 textbook: torch RMSNorm, then RoPE as a complex rotation of the two halves."""
    xn = torch.nn.functional.rms_norm(torch.tensor(x, dtype=torch.float64), (128,),
                                      torch.tensor(w, dtype=torch.float64), eps=1e-6).numpy()
    z = (xn[..., :64] + 1j * xn[..., 64:]) * (c + 1j * s)
    return np.concatenate([z.real, z.imag], axis=-1)


def test_prefill_norm_rope_matches_float64():
    rng = np.random.default_rng(5)
    gen = torch.Generator().manual_seed(1)
    N, hq, hkv = 37, 16, 8
    q = (3 * torch.randn(N, hq, 128, generator=gen)).bfloat16().float().numpy()
    k = torch.randn(N, hkv, 128, generator=gen).bfloat16().float().numpy()
    qw = (1 + 0.1 * torch.randn(128, generator=gen)).bfloat16().float().numpy()
    kw = (1 + 0.1 * torch.randn(128, generator=gen)).bfloat16().float().numpy()
    ang = rng.uniform(0, 1000, (N, 1, 64))
    cos = torch.tensor(np.cos(ang)).bfloat16().float().numpy()
    sin = torch.tensor(np.sin(ang)).bfloat16().float().numpy()
    qo, ko = okv.fused_norm_rope_prefill(q, k, qw, kw, cos, sin, 1e-6)
    assert qo.shape == q.shape and ko.shape == k.shape
    # each output is one bf16 rounding (relative 2^-9) of the float64 value, up to the fp32
    # steps before it
    for out, x, w in ((qo, q, qw), (ko, k, kw)):
        ref = _norm_rope64(x, w, cos, sin)
        assert np.all(np.abs(out - ref) <= 2 ** -8 * np.abs(ref) + 1e-6)
    assert np.array_equal(qo, bf16_round(qo))  # bf16-representable


def test_prefill_norm_rope_known_answers():
    # a constant row c normalizes to sign(c) (up to eps); zero angle is the identity and a
    # quarter turn maps (x1, x2) to (-x2, x1)
    N = 2
    x = np.zeros((N, 1, 128), np.float32)
    x[0, 0, :] = 3.0
    x[1, 0, :64], x[1, 0, 64:] = 1.0, -2.0
    w = np.full(128, 0.5, np.float32)
    cos = np.zeros((N, 1, 64), np.float32)
    sin = np.zeros((N, 1, 64), np.float32)
    cos[0], sin[1] = 1.0, 1.0
    qo, ko = okv.fused_norm_rope_prefill(x, x, w, w, cos, sin, 0.0)
    assert np.array_equal(qo, ko)
    assert np.all(qo[0, 0] == F32(0.5))
    # token 1: rms = sqrt((1 + 4) / 2), x1n = 0.5 / rms, x2n = -1 / rms; rotated: (-x2n, x1n)
    rms = np.sqrt(2.5)
    assert np.allclose(qo[1, 0, :64], 1.0 / rms, rtol=2 ** -8)
    assert np.allclose(qo[1, 0, 64:], 0.5 / rms, rtol=2 ** -8)


def test_prefill_norm_rope_is_the_decode_rotation():
    # the decode write's q (before the calibration fold) and the prefill op share the math: with
    # calibration ones the decode q_out equals the prefill q_out for the same rows
    gen = torch.Generator().manual_seed(2)
    B, hq, hkv = 4, 16, 8
    q = torch.randn(B, hq, 128, generator=gen).bfloat16().float().numpy()
    k = torch.randn(B, hkv, 128, generator=gen).bfloat16().float().numpy()
    w = (1 + 0.1 * torch.randn(128, generator=gen)).bfloat16().float().numpy()
    ang = np.random.default_rng(6).uniform(0, 50, (B, 1, 64))
    cos = torch.tensor(np.cos(ang)).bfloat16().float().numpy()
    sin = torch.tensor(np.sin(ang)).bfloat16().float().numpy()
    cache = okv.CacheArrays.empty(B, hkv, 4, 128)
    qd = okv.fused_rope_kv_decode(q, k, k, w, w, cos, sin, np.arange(B), cache,
                                  np.zeros(B, np.int64), B, 1e-6)
    qp, _ = okv.fused_norm_rope_prefill(q, k, w, w, cos, sin, 1e-6)
    assert np.array_equal(qd, qp)


def test_butterfly_sum_is_a_sum():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((100, 64)).astype(np.float32)
    assert np.allclose(butterfly_sum64(x), x.astype(np.float64).sum(axis=1), rtol=1e-5, atol=1e-5)
    assert butterfly_sum64(np.arange(64, dtype=np.float32)) == F32(2016.0)


def test_dequantize_prefix_known_answer():
    cache = okv.CacheArrays.empty(3, 2, 8, 128)
    cache.k[1, :, :4] = np.arange(-64, 64, dtype=np.int8)[None, None, :]
    cache.v[1, :, :4] = np.arange(63, -65, -1, dtype=np.int8)[None, None, :]
    cache.k_scale[1, :, :4] = 0.25
    cache.v_scale[1, :, :4] = 2.0
    cache.k_calibration[1, :, 0] = 4.0
    ko, vo = okv.dequantize_kv_prefix(cache, np.array([0, 0, 4]), np.array([0, 1]))
    assert ko.shape == (2, 4, 128)
    assert np.array_equal(ko[0, 0], np.arange(-64, 64, dtype=np.float32))  # q * 0.25 * 4
    assert np.array_equal(vo[1, 3], 2.0 * np.arange(63, -65, -1, dtype=np.float32))


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(100000) * 10.0 ** rng.integers(-30, 30, 100000)).astype(np.float32)
    x[:4] = [np.inf, -np.inf, 0.0, -0.0]
    ref = torch.tensor(x).bfloat16().float().numpy()
    assert np.array_equal(bf16_round(x).view(np.uint32), ref.view(np.uint32))
