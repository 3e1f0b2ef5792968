"""Shared test helpers: moving caches between torch and the numpy oracle, tolerance checks."""

import sys

import numpy as np
import torch

from oracle import kv_cache as okv

TOL_MAX, TOL_MEAN = 2e-2, 2e-3  # bf16 attention tolerance of the north star


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def cache_np(c) -> okv.CacheArrays:
    return okv.CacheArrays(*(t.detach().cpu().numpy().copy() for t in
                             (c.k, c.v, c.k_scale, c.v_scale, c.k_calibration)))


def cache_to(c, device, LayerKVCache):
    return LayerKVCache(*(t.to(device).clone() for t in
                          (c.k, c.v, c.k_scale, c.v_scale, c.k_calibration)))


def assert_cache_bitwise(gpu_cache, ref: okv.CacheArrays, what=""):
    got = cache_np(gpu_cache)
    for name in ("k", "v", "k_scale", "v_scale", "k_calibration"):
        a, b = getattr(got, name), getattr(ref, name)
        if a.dtype == np.float32:
            a, b = a.view(np.uint32), b.view(np.uint32)
        bad = np.argwhere(a != b)
        assert bad.size == 0, f"{what} {name}: {len(bad)} mismatches, first at {bad[:4].tolist()}"


def rel_err(got, ref):
    """|got - ref| of each output vector (the last axis) divided by that vector's largest |ref|:
    the bf16 tolerance made independent of the output's magnitude."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.maximum(np.abs(ref).max(axis=-1, keepdims=True), np.finfo(np.float32).tiny)
    return np.abs(got - ref) / scale


def assert_attn_close(got, ref, what="", rel=True, abs_scale=1.0):
    """The north star's bf16 attention tolerance (max abs <= 2e-2, mean abs <= 2e-3) on
    unit-scale data, and the same bounds on the scale-normalised error (rel_err), so that an
    error that grows with the output's magnitude cannot hide behind small outputs. abs_scale
    multiplies the absolute bounds for data that is not unit-scale (V scaled by 1e2, or peaked
    attention whose outputs are single V rows of magnitude up to ~4, where one bf16 rounding
    step of an output is already 2^-6); the scale-normalised bounds do not change."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err = np.abs(got - ref)
    r = rel_err(got, ref)
    say(f"{what}: max abs err {err.max():.3e} mean {err.mean():.3e}; "
        f"scaled max {r.max():.3e} mean {r.mean():.3e}")
    assert err.max() <= TOL_MAX * abs_scale and err.mean() <= TOL_MEAN * abs_scale, what
    if rel:
        assert r.max() <= TOL_MAX and r.mean() <= TOL_MEAN, f"{what} (scale-normalised)"


def bf16_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


PLAN_FIELDS = ("found", "sb", "hk", "piece", "npieces", "kt_begin", "kt_end", "npt", "nct", "r0",
               "r1", "seq_start", "P", "slot", "straddle", "item_base")


def prefill_plan(native, g) -> np.ndarray:
    """The prefill launch's work list for the device-resident mixed workload `g`, as the kernel's
    own schedule computes it (ie_prefill_attention_plan through the C ABI): one row per
    workgroup of the launch, fields PLAN_FIELDS ("hk" is the work unit: KV head x query-head
    pair, the KV head itself at GQA 2); only rows with found == 1 carry work."""
    import ctypes

    lib = native.cabi()
    gi = g.inputs
    ts = gi["tile_start"]
    hq, hkv = g.q.shape[1], g.cache.k.shape[1]
    grid = lib.ie_prefill_attention_grid(ctypes.c_int32(ts.shape[0]), ctypes.c_int32(g.block_m),
                                         ctypes.c_int32(hq), ctypes.c_int32(hkv))
    rows = torch.full((grid, 16), -7, dtype=torch.int32, device=ts.device)
    fn = lib.ie_prefill_attention_plan
    fn.restype = ctypes.c_int
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = fn(p(gi["seq_ids"]), p(gi["cu_seqlens"]), p(ts), ctypes.c_int32(ts.shape[0]),
            ctypes.c_int32(g.block_m), ctypes.c_int64(g.q.shape[0]), ctypes.c_int32(hq),
            ctypes.c_int32(hkv),
            p(gi["slot_ids"]), p(gi["cu_cached"]), ctypes.c_int32(gi["slot_ids"].shape[0]),
            p(rows), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, lib.ie_attn_last_error()
    torch.cuda.synchronize()
    return rows.cpu().numpy()
