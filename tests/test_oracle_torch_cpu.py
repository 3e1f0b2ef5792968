"""The PyTorch-on-CPU restatement used as the benchmark's CPU baseline (oracle/torch_cpu.py),
pinned against the numpy oracle and the float64 textbook forms (CPU only)."""

import numpy as np
import torch

from helpers import cache_np
from oracle import attention as oat
from oracle import kv_cache as okv
from oracle import torch_cpu as otc

SCALE = 128 ** -0.5


def test_decode_matches_float64(workloads):
    ctx = [5, 300, 300, 300, 1, 4096, 4096, 77] + [64] * 20
    wl = workloads.decode_workload(ctx, seed=3, num_decoding=26)
    c = wl.cache
    got = otc.decode_attention(wl.q, c.k, c.v, c.k_scale, c.v_scale, wl.cached_lens, wl.slot_ids,
                               26, SCALE).numpy()
    want = oat.decode_attention_f64(wl.q.float().numpy(), cache_np(c), wl.cached_lens.numpy(),
                                    wl.slot_ids.numpy(), 26, SCALE)[:26]
    assert np.abs(got - want).max() < 2e-5


def test_quantize_matches_oracle_bitwise(workloads):
    wl = workloads.mixed_workload([9, 3], [(40, 0), (7, 33), (130, 200), (0, 5)], seed=4,
                                  max_len=512)
    ins = {n: t.numpy() for n, t in wl.inputs.items()}
    ref = cache_np(wl.cache)
    okv.quantize_kv_prefill(wl.k.float().numpy(), wl.v.float().numpy(), ins["cu_seqlens"],
                            ins["slot_ids"], ins["cached_lens"], int(ins["num_decoding"][0]), ref)
    c = wl.cache
    gi = wl.inputs
    otc.quantize_kv_prefill(wl.k, wl.v, gi["cu_seqlens"], gi["slot_ids"], gi["cached_lens"],
                            int(gi["num_decoding"][0]), c.k, c.v, c.k_scale, c.v_scale,
                            c.k_calibration)
    got = cache_np(c)
    for name in ("k", "v", "k_scale", "v_scale", "k_calibration"):
        a, b = getattr(got, name), getattr(ref, name)
        if a.dtype == np.float32:
            a, b = a.view(np.uint32), b.view(np.uint32)
        assert np.array_equal(a, b), name


def test_prefill_matches_float64(workloads):
    wl = workloads.mixed_workload([9, 3], [(40, 0), (7, 33), (130, 200)], seed=5, block_m=32,
                                  max_len=512)
    ins = {n: t.numpy() for n, t in wl.inputs.items()}
    c = wl.cache
    got = otc.prefill_attention(wl.q, wl.k, wl.v, wl.inputs["cu_seqlens"], wl.inputs["slot_ids"],
                                wl.inputs["cu_cached"], int(ins["num_decoding"][0]), c.k, c.v,
                                c.k_scale, c.v_scale, c.k_calibration).numpy()
    # float64 dequantized prefix (no bf16 rounding), then the textbook causal form
    cn = cache_np(c)
    hkv, total = 8, int(ins["cu_cached"][-1])
    kp = np.zeros((hkv, total, 128))
    vp = np.zeros((hkv, total, 128))
    for e in range(len(ins["slot_ids"])):
        p0, p1 = int(ins["cu_cached"][e]), int(ins["cu_cached"][e + 1])
        s = int(ins["slot_ids"][e])
        n = p1 - p0
        kp[:, p0:p1] = (cn.k[s, :, :n] * cn.k_scale[s, :, :n, None].astype(np.float64)
                        * cn.k_calibration[s, :, 0][:, None, :])
        vp[:, p0:p1] = cn.v[s, :, :n] * cn.v_scale[s, :, :n, None].astype(np.float64)
    want = oat.prefill_attention_f64(wl.q.float().numpy(), wl.k.float().numpy(),
                                     wl.v.float().numpy(), ins["cu_seqlens"], ins["tile_start"],
                                     wl.block_m, kp, vp, ins["cu_cached"])
    rows = ~np.isnan(want[:, 0, 0])
    assert rows.sum() == 40 + 7 + 130
    assert np.abs(got[rows] - want[rows]).max() < 2e-5
