"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py from the oracle).

CPU: the oracle still reproduces every fixture (bit-exact for int8 values, scales and bf16 bits;
1e-6 for fp32 attention outputs, whose BLAS summation order may differ between machines), and the
attention fixtures agree with the float64 textbook forms within the bf16 tolerance.
GPU: the HIP path, through the torch ops, on the fixtures' inputs: bit-exact for the cache writes,
the decode q and the prefill q/k norm + rope, within the attention tolerance for decode and
prefill attention."""

from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import assert_attn_close, bf16_np, cache_np, say
from oracle import attention as oat
from oracle import kv_cache as okv
from oracle.numerics import bf16_bits, bits_to_f32

GOLD = Path(__file__).resolve().parent / "golden"
SCALE = 128 ** -0.5


def load(name):
    with np.load(GOLD / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def arrays(d, prefix):
    cal = f"{prefix}_k_cal" if f"{prefix}_k_cal" in d else f"{prefix}_k_calibration"
    return okv.CacheArrays(d[f"{prefix}_k"].copy(), d[f"{prefix}_v"].copy(),
                           d[f"{prefix}_k_scale"].copy(), d[f"{prefix}_v_scale"].copy(),
                           d[cal].copy())


def f32(bits):
    return bits_to_f32(bits)


def bitwise_equal(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == np.float32:
        a, b = a.view(np.uint32), b.view(np.uint32)
    return a.shape == b.shape and np.array_equal(a, b)


# ------------------------------------------------------------------------------------------
# CPU: the oracle against the fixtures
# ------------------------------------------------------------------------------------------

def test_fixture_quant_rows():
    d = load("quant_rows")
    q, s = okv.quantize_rows(d["rows"])
    assert bitwise_equal(q, d["q"]) and bitwise_equal(s, d["s"])
    assert d["q"][1, 5] == 127 and d["q"][0].max() == 0  # one-hot, zero row
    assert list(d["q"][4, :4]) == [127, 64, 0, 2]  # s == 1: ties to even


def test_fixture_prefill_write():
    d = load("prefill_write")
    c = okv.CacheArrays(*(d[f"before_{n}"].copy() for n in
                          ("k", "v", "k_scale", "v_scale", "k_calibration")))
    okv.quantize_kv_prefill(f32(d["k_bits"]), f32(d["v_bits"]), d["in_cu_seqlens"],
                            d["in_slot_ids"], d["in_cached_lens"], int(d["in_num_decoding"][0]), c)
    for n in ("k", "v", "k_scale", "v_scale", "k_calibration"):
        assert bitwise_equal(getattr(c, n), d[f"after_{n}"]), n


def _rope_inputs(d):
    qkv = f32(d["qkv_bits"])
    B = qkv.shape[0]
    return (qkv[:, :2048].reshape(B, 16, 128), qkv[:, 2048:3072].reshape(B, 8, 128),
            qkv[:, 3072:].reshape(B, 8, 128))


def test_fixture_rope_kv_decode():
    d = load("rope_kv_decode")
    q, k, v = _rope_inputs(d)
    B = q.shape[0]
    pool, L = d["after_k"].shape[0], d["after_k"].shape[2]
    c = okv.CacheArrays(np.zeros((pool, 8, L, 128), np.int8), np.zeros((pool, 8, L, 128), np.int8),
                        np.zeros((pool, 8, L), np.float32), np.zeros((pool, 8, L), np.float32),
                        d["cal"].copy())
    q_out = okv.fused_rope_kv_decode(q, k, v, f32(d["qw_bits"]), f32(d["kw_bits"]),
                                     f32(d["cos_bits"]), f32(d["sin_bits"]), d["slot_ids"], c,
                                     d["cached_lens"], B, 1e-6)
    assert np.array_equal(bf16_bits(q_out), d["q_out_bits"])
    for n in ("k", "v", "k_scale", "v_scale"):
        assert bitwise_equal(getattr(c, n), d[f"after_{n}"]), n


def test_fixture_norm_rope_prefill():
    d = load("norm_rope_prefill")
    qkv = f32(d["qkv_bits"])
    N = qkv.shape[0]
    qo, ko = okv.fused_norm_rope_prefill(qkv[:, :2048].reshape(N, 16, 128),
                                         qkv[:, 2048:3072].reshape(N, 8, 128), f32(d["qw_bits"]),
                                         f32(d["kw_bits"]), f32(d["cos_bits"]),
                                         f32(d["sin_bits"]), 1e-6)
    assert np.array_equal(bf16_bits(qo), d["q_out_bits"])
    assert np.array_equal(bf16_bits(ko), d["k_out_bits"])


def test_fixture_decode_config1():
    d = load("decode_config1")
    c = arrays(d, "cache")
    args = (f32(d["q_bits"]), c, d["cached_lens"], d["slot_ids"], 1, SCALE)
    out = oat.decode_attention(*args)
    np.testing.assert_allclose(out, d["out"], rtol=0, atol=1e-6)
    ref64 = oat.decode_attention_f64(*args)
    assert np.abs(d["out"] - ref64).max() <= 2e-2


def test_fixture_prefill_small():
    d = load("prefill_small")
    c = arrays(d, "cache")
    kp, vp = okv.dequantize_kv_prefix(c, d["in_cu_cached"], d["in_slot_ids"])
    args = (f32(d["q_bits"]), f32(d["k_bits"]), f32(d["v_bits"]), d["in_cu_seqlens"],
            d["in_tile_start"], int(d["block_m"]), kp, vp, d["in_cu_cached"])
    out = oat.prefill_attention(*args)
    cov = ~np.isnan(d["out"][:, 0, 0])
    assert cov.sum() == 31  # the two chunks' rows; decoder rows are not prefill's
    np.testing.assert_allclose(out[cov], d["out"][cov], rtol=0, atol=1e-6)
    ref64 = oat.prefill_attention_f64(*args)
    assert np.abs(d["out"][cov] - ref64[cov]).max() <= 2e-2


# ------------------------------------------------------------------------------------------
# GPU: the HIP path against the fixtures
# ------------------------------------------------------------------------------------------

def _t(a, dev):
    a = np.asarray(a)
    if a.dtype == np.uint16:  # bf16 bits
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16).to(dev)
    return torch.from_numpy(a.copy()).to(dev)


def _cache(ie, c: okv.CacheArrays, dev):
    return ie.kernels.LayerKVCache(*(_t(getattr(c, n), dev) for n in
                                     ("k", "v", "k_scale", "v_scale", "k_calibration")))


@pytest.mark.gpu
def test_gpu_quant_rows(ie, dev):
    """The 16 fixture rows as K and V of one chunk written after one cached token (stored
    calibration 1): the cache holds exactly the fixture's int8 rows and scales."""
    say("golden quant_rows through quantize_kv_prefill")
    d = load("quant_rows")
    rows_bits = bf16_bits(d["rows"])
    n = rows_bits.shape[0]
    kb = np.broadcast_to(rows_bits[:, None, :], (n, 8, 128)).copy()
    vb = np.broadcast_to(rows_bits[(np.arange(n) + 3) % n][:, None, :], (n, 8, 128)).copy()
    cache = ie.make_layer_cache(2, 8, 32, 128, device=dev)
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=dev)
    ie.quantize_kv_prefill(_t(kb, dev), _t(vb, dev), i32([0, n]), i32([1]), i32([1]), i32([0]),
                           cache)
    torch.cuda.synchronize()
    got = cache_np(cache)
    for h in range(8):
        assert bitwise_equal(got.k[1, h, 1:1 + n], d["q"])
        assert bitwise_equal(got.k_scale[1, h, 1:1 + n], d["s"])
        assert bitwise_equal(got.v[1, h, 1:1 + n], d["q"][(np.arange(n) + 3) % n])
    assert not got.k[1, :, 0].any() and not got.k[0].any()  # column 0 and slot 0 untouched


@pytest.mark.gpu
def test_gpu_prefill_write(ie, dev):
    say("golden prefill_write")
    d = load("prefill_write")
    before = okv.CacheArrays(*(d[f"before_{n}"] for n in
                               ("k", "v", "k_scale", "v_scale", "k_calibration")))
    cache = _cache(ie, before, dev)
    ie.quantize_kv_prefill(_t(d["k_bits"], dev), _t(d["v_bits"], dev), _t(d["in_cu_seqlens"], dev),
                           _t(d["in_slot_ids"], dev), _t(d["in_cached_lens"], dev),
                           _t(d["in_num_decoding"], dev), cache)
    torch.cuda.synchronize()
    got = cache_np(cache)
    for n in ("k", "v", "k_scale", "v_scale", "k_calibration"):
        assert bitwise_equal(getattr(got, n), d[f"after_{n}"]), n


@pytest.mark.gpu
def test_gpu_rope_kv_decode(ie, dev):
    say("golden rope_kv_decode")
    d = load("rope_kv_decode")
    qkv = _t(d["qkv_bits"], dev)
    B = qkv.shape[0]
    pool, L = d["after_k"].shape[0], d["after_k"].shape[2]
    cache = ie.make_layer_cache(pool, 8, L, 128, device=dev)
    cache.k_calibration.copy_(_t(d["cal"], dev))
    q_out = ie.fused_rope_kv_decode(
        qkv[:, :2048].view(B, 16, 128), qkv[:, 2048:3072].view(B, 8, 128),
        qkv[:, 3072:].view(B, 8, 128), _t(d["qw_bits"], dev), _t(d["kw_bits"], dev),
        _t(d["cos_bits"], dev), _t(d["sin_bits"], dev), _t(d["slot_ids"], dev), cache,
        _t(d["cached_lens"], dev), torch.tensor([B], dtype=torch.int32, device=dev), 1e-6)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(bf16_np(q_out)), d["q_out_bits"])
    got = cache_np(cache)
    for n in ("k", "v", "k_scale", "v_scale"):
        assert bitwise_equal(getattr(got, n), d[f"after_{n}"]), n


@pytest.mark.gpu
def test_gpu_norm_rope_prefill(ie, dev):
    say("golden norm_rope_prefill")
    d = load("norm_rope_prefill")
    qkv = _t(d["qkv_bits"], dev)
    N = qkv.shape[0]
    q_out, k_out = ie.fused_norm_rope_prefill(
        qkv[:, :2048].view(N, 16, 128), qkv[:, 2048:3072].view(N, 8, 128), _t(d["qw_bits"], dev),
        _t(d["kw_bits"], dev), _t(d["cos_bits"], dev), _t(d["sin_bits"], dev), 1e-6)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_bits(bf16_np(q_out)), d["q_out_bits"])
    assert np.array_equal(bf16_bits(bf16_np(k_out)), d["k_out_bits"])


@pytest.mark.gpu
def test_gpu_decode_config1(ie, dev):
    say("golden decode_config1")
    d = load("decode_config1")
    cache = _cache(ie, arrays(d, "cache"), dev)
    out = ie.decode_attention(_t(d["q_bits"], dev), cache, _t(d["cached_lens"], dev),
                              _t(d["slot_ids"], dev),
                              torch.tensor([1], dtype=torch.int32, device=dev), SCALE)
    torch.cuda.synchronize()
    assert_attn_close(bf16_np(out), d["out"], "golden decode config 1")


@pytest.mark.gpu
def test_gpu_prefill_small(ie, dev):
    say("golden prefill_small")
    d = load("prefill_small")
    cache = _cache(ie, arrays(d, "cache"), dev)
    g = lambda n: _t(d[f"in_{n}"], dev)
    out = ie.prefill_attention(_t(d["q_bits"], dev), _t(d["k_bits"], dev), _t(d["v_bits"], dev),
                               g("seq_ids"), g("cu_seqlens"), g("tile_start"), cache,
                               g("slot_ids"), g("cu_cached"), int(d["block_m"]))
    torch.cuda.synchronize()
    cov = ~np.isnan(d["out"][:, 0, 0])
    assert_attn_close(bf16_np(out)[cov], d["out"][cov], "golden prefill small")
