"""Benchmark of the int8-KV attention hot path on one MI355X.

Headline (BASELINE metric): split-K int8-KV decode attention at B=64, ctx=4096, Hq=16, Hkv=8,
D=128 — µs per layer and achieved HBM GB/s against the 8 TB/s peak. One step = one
`decode_attention` call over the whole batch (one launch: split-K pieces, the last piece of
each sequence merging them), inputs resident in HBM. Distinct cache sets are rotated between steps so the 256 MB MALL cannot serve a repeat.

Also reported beside it (extra keys): config-4 KV quantize-on-write, chunked-prefill attention,
the prefill q/k RMSNorm + RoPE of its 1,024 packed tokens and the whole config-4 attention step,
token sampling and the projection GEMMs at config 5's shape, each timed with HIP events on the
stream the kernels run on; the CPU baseline (the same math in PyTorch on the host cores) for
the headline, the config-4 KV write and the config-4 prefill; and config 5: a whole
greedy decode step of a Qwen3-1.7B-shaped model (28 layers, random weights, B=32, ctx ~
U[128, 4096)) replayed as a hipGraph, with the share of the step spent in the attention kernels
(the same kernels captured alone).

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-step] [--sweep]
"""

import argparse
import importlib
import json
import os
import sys
import time
from pathlib import Path

import torch

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

METRIC = "int8-KV decode attn µs/layer + HBM GB/s (% of 8 TB/s), B=64 ctx=4096"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2516.6
SCALE = 128 ** -0.5


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _events(n):
    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


def time_decode(ie, wls, steps, warmup):
    """Whole-step time: `decode_attention` back to back between two events, cycling through the
    cache sets. The op is one launch (decode_attention_kernel, whose last piece per sequence also
    merges the pieces), so this is also that kernel's average duration."""
    K = ie.kernels
    outs = [torch.empty_like(w.q) for w in wls]

    def run(i):
        w = wls[i % len(wls)]
        K.decode_attention(w.q, w.cache, w.cached_lens, w.slot_ids, w.num_decoding, SCALE,
                           out=outs[i % len(wls)])

    for i in range(warmup):
        run(i)
    torch.cuda.synchronize()
    e0, e1 = _events(2)
    e0.record()
    for i in range(steps):
        run(i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


SETTLE_S = 0.15  # minimum warm-up wall time of an extra line (--settle-ms)


def settle(fn):
    """Keeps calling fn until SETTLE_S seconds have passed since the first call. After a second
    of idle the device's clocks need tens of milliseconds of load to come back up: a 241 µs
    prefill ran its first 25 calls at 290 µs on average and reached 241 µs only after ~150 calls,
    so a few warm-up calls leave the timed calls in the ramp."""
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < SETTLE_S:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()


def time_op(fn, steps, warmup):
    """Average time of back-to-back calls between two events: events around every call of a
    microsecond-scale kernel would add several microseconds of their own per call. Warm-up: the
    `warmup` calls, then more until SETTLE_S seconds have passed (untimed)."""
    for _ in range(warmup):
        fn()
    settle(fn)
    torch.cuda.synchronize()
    e0, e1 = _events(2)
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def bench_norm_rope(K, N, steps, warmup, dev):
    """fused_norm_rope_prefill over N packed tokens whose q/k are strided views of a fused qkv
    row (Qwen3-1.7B: 16 + 8 + 8 heads of 128). Algorithmic bytes: q and k read and written once
    (bf16), plus the per-token cos/sin rows."""
    g = torch.Generator().manual_seed(0)
    qkv = torch.randn(N, 32 * 128, generator=g).bfloat16().to(dev)
    w = (1 + 0.1 * torch.randn(2, 128, generator=g)).bfloat16().to(dev)
    ang = torch.rand(N, 1, 64, generator=g) * 1000
    cos, sin = ang.cos().bfloat16().to(dev), ang.sin().bfloat16().to(dev)
    q, k = qkv[:, :2048].view(N, 16, 128), qkv[:, 2048:3072].view(N, 8, 128)
    op = lambda: K.fused_norm_rope_prefill(q, k, w[0], w[1], cos, sin, 1e-6)
    ms = time_op(op, steps, warmup)
    gms = time_graph(op)
    nbytes = N * 24 * 128 * 2 * 2 + N * 64 * 2 * 2
    return {"us": round(ms * 1e3, 3), "us_graph": round(gms * 1e3, 3),
            "GBps_graph": round(nbytes / (gms * 1e-3) / 1e9, 1), "bytes": nbytes, "tokens": N}


def time_graph(fn, calls=20, reps=5):
    """Average time per call of `calls` back-to-back calls captured in one hipGraph and replayed:
    the GPU-side time of a µs-scale op without the host's per-call launch cost (an eager loop
    of such calls measures the host as much as the kernels)."""
    fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):  # the warmed-up stream: its workspaces exist
        for _ in range(calls):
            fn()
    settle(g.replay)
    e0, e1 = _events(2)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (reps * calls)


def bench_sample(K, B, V, steps, warmup, dev):
    """`sample` over bf16 logits [B, V] (Qwen3-1.7B: V = 151,936): greedy (tau 0, one read of
    the logits: B * V * 2 bytes) and Gumbel-max at tau 1 (the same bytes plus a Philox draw and
    two logarithms per entry)."""
    g = torch.Generator().manual_seed(0)
    logits = (2 * torch.randn(B, V, generator=g)).bfloat16().to(dev)
    seed = torch.zeros(1, dtype=torch.int64, device=dev)
    nbytes = B * V * 2
    res = {"batch": B, "vocab": V, "bytes": nbytes}
    for tau in (0.0, 1.0):
        op = lambda: K.sample(logits, tau, seed)
        ms = time_op(op, steps, warmup)
        gms = time_graph(op)
        res[f"tau{tau:g}"] = {"us": round(ms * 1e3, 3), "us_graph": round(gms * 1e3, 3),
                              "GBps_graph": round(nbytes / (gms * 1e-3) / 1e9, 1)}
    return res


def bench_linear(K, M, dev):
    """skinny_matmul (best n_tiles) and the library GEMM on Qwen3-1.7B's projection shapes at M
    rows, each timed over weight copies that together exceed the 256 MB last-level cache (the
    weights come from HBM, as every layer's do in a step), and the best of the launches on the
    weight in fragment order (swizzle_weight at each 16-row tile width; the LM head then runs one
    looping workgroup per CU). Algorithmic bytes: the weight."""
    import math
    shapes = {"qkv": (4096, 2048), "o_proj": (2048, 2048), "gate_up": (12288, 2048),
              "down": (2048, 6144), "lm_head": (151_936, 2048)}
    res = {"rows": M}
    g = torch.Generator().manual_seed(0)
    for name, (N, Kd) in shapes.items():
        nbytes = N * Kd * 2
        ws = [(0.02 * torch.randn(N, Kd, generator=g)).bfloat16().to(dev)
              for _ in range(max(1, math.ceil((512 << 20) / nbytes)))]
        x = torch.randn(M, Kd, generator=g).bfloat16().to(dev)
        calls = lambda f: [lambda w=w: f(w) for w in ws] * max(1, 16 // len(ws))
        lib_ms = time_graph_calls(calls(lambda w: torch.nn.functional.linear(x, w)))
        best = None
        for nt in (0, 1, 2, 4):
            if N % (16 * max(1, nt)) == 0:
                t = time_graph_calls(calls(lambda w, nt=nt: K.skinny_matmul(x, w, nt)))
                best = (t, nt) if best is None or t < best[0] else best
        res[name] = {"bytes": nbytes, "skinny_us": round(best[0] * 1e3, 2), "n_tiles": best[1],
                     "skinny_GBps": round(nbytes / (best[0] * 1e-3) / 1e9, 1),
                     "library_us": round(lib_ms * 1e3, 2),
                     "library_GBps": round(nbytes / (lib_ms * 1e-3) / 1e9, 1)}
        sbest = None  # the launch on the weight in fragment order (swizzle_weight), each width
        for nt in (1, 2, 4):
            if N % (16 * nt) or nt + -(-M // 16) > 6:
                continue
            sws = [K.swizzle_weight(w, nt) for w in ws]
            scalls = [lambda w=w: K.skinny_matmul(x, w, nt, swizzled=True)
                      for w in sws] * max(1, 16 // len(sws))
            t = time_graph_calls(scalls)
            sbest = (t, nt) if sbest is None or t < sbest[0] else sbest
            del sws
        if sbest is not None:
            res[name]["swizzled_us"] = round(sbest[0] * 1e3, 2)
            res[name]["swizzled_n_tiles"] = sbest[1]
            res[name]["swizzled_GBps"] = round(nbytes / (sbest[0] * 1e-3) / 1e9, 1)
        del ws
    return res


def time_graph_calls(fns, reps=3):
    """Average time per call of the calls `fns` captured in order in one hipGraph."""
    for f in fns[:2]:
        f()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fns[0]()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for f in fns:
            f()
    settle(g.replay)
    e0, e1 = _events(2)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (reps * len(fns))


def cpu_threads() -> int:
    """Host threads for the CPU baseline: the cores this process may run on, capped by the
    box's OMP_NUM_THREADS share when one is set."""
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    return min(n, int(omp)) if omp.isdigit() and int(omp) > 0 else n


def _repeat(fn, min_seconds):
    fn()  # first call: allocator and thread-pool warm-up, not timed
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds and reps >= 2:
            return dt / reps, dt, reps


def cpu_baselines(wl_gpu, alg_bytes, W, min_seconds):
    """The reference attention math restated in PyTorch (oracle/torch_cpu.py: fp32 dequant,
    scores, softmax, PV; batches in slices of <= 16 sequences) on the host cores, on the same
    kind of inputs: the headline decode batch (its 64 cache rows copied to host memory), and
    config 4's KV write and chunked-prefill attention. Each is repeated for at least
    `min_seconds` (the decode sample) or a third of it (the two config-4 ops)."""
    from oracle import torch_cpu as otc

    threads = cpu_threads()
    torch.set_num_threads(threads)
    B = len(wl_gpu.ctx)
    slots = wl_gpu.slot_ids.long()
    c = wl_gpu.cache
    k, v, ks, vs = (t[slots].cpu() for t in (c.k, c.v, c.k_scale, c.v_scale))
    q = wl_gpu.q.cpu()
    lens = wl_gpu.cached_lens.cpu()
    rows = torch.arange(B, dtype=torch.int32)
    per, dt, reps = _repeat(lambda: otc.decode_attention(q, k, v, ks, vs, lens, rows, B, SCALE),
                            min_seconds)
    res = {"value": round(alg_bytes / per / 1e9, 3), "unit": "GB/s",
           "us_per_layer": round(per * 1e6, 1), "cores": threads, "kind": "port",
           "sample": f"the whole headline batch ({B} sequences at ctx {wl_gpu.ctx[0]}, "
                     f"slices of {otc.SLICE}), {reps} passes in {dt:.1f} s",
           "cpu": _cpu_model(), "torch_threads": torch.get_num_threads()}
    del k, v, ks, vs
    mw = W.config4(seed=0)
    gi = mw.inputs
    nd = int(gi["num_decoding"][0])
    cache = mw.cache
    kv_per, kv_dt, kv_reps = _repeat(lambda: otc.quantize_kv_prefill(
        mw.k, mw.v, gi["cu_seqlens"], gi["slot_ids"], gi["cached_lens"], nd, cache.k, cache.v,
        cache.k_scale, cache.v_scale, cache.k_calibration), min_seconds / 3)
    n_new = sum(L for L, _ in mw.chunks)
    kv_bytes = n_new * 8 * (128 * 2 * 2 + 128 * 2 + 8)
    res["kv_write_config4"] = {"us": round(kv_per * 1e6, 1),
                               "GBps": round(kv_bytes / kv_per / 1e9, 3),
                               "sample": f"{kv_reps} calls in {kv_dt:.1f} s"}
    pf_per, pf_dt, pf_reps = _repeat(lambda: otc.prefill_attention(
        mw.q, mw.k, mw.v, gi["cu_seqlens"], gi["slot_ids"], gi["cu_cached"], nd, cache.k,
        cache.v, cache.k_scale, cache.v_scale, cache.k_calibration), min_seconds / 3)
    flops = W.prefill_flops(mw.chunks)
    res["prefill_config4"] = {"us": round(pf_per * 1e6, 1),
                              "GFLOPs": round(flops / pf_per / 1e9, 1),
                              "sample": f"{pf_reps} calls in {pf_dt:.1f} s"}
    return res


def bench_mixed_step(W, dev):
    """Config 4 as one attention step (qwen3-1.7b/architecture.py:124-197 through
    attention_layer.attention: prefill norm/RoPE of all 1,054 rows, KV quantize-on-write,
    prefill attention over the int8 prefix, decode norm/RoPE/write and decode attention of the
    30 decoders into the same output), captured as a hipGraph and replayed."""
    al = importlib.import_module("inference-engine_amd.attention_layer")
    wl = W.mixed_to(W.config4(seed=0), dev)
    gi = wl.inputs
    N = wl.q.shape[0]
    g = torch.Generator().manual_seed(0)
    qkv = torch.randn(N, 32 * 128, generator=g).bfloat16().to(dev)
    q, k, v = qkv[:, :2048].view(N, 16, 128), qkv[:, 2048:3072].view(N, 8, 128), \
        qkv[:, 3072:].view(N, 8, 128)
    w = torch.ones(2, 128, dtype=torch.bfloat16, device=dev)
    cos, sin = al.rope_tables(gi["positions"], al.rope_inv_freq(128, 1e6, dev))
    ps = al.PrefixScratch(None, None, gi["cu_cached"])
    op = lambda plan=None, dplan=None: al.attention(
        q, k, v, gi["seq_ids"], gi["cu_seqlens"], cos, sin, wl.cache, gi["cached_lens"],
        gi["slot_ids"], gi["tile_start"], wl.block_m, ps, gi["num_decoding"], w[0], w[1], 1e-6,
        plan, dplan)
    ms = time_graph(op)
    K = importlib.import_module("inference-engine_amd.kernels")
    plan = K.prefill_plan(gi["seq_ids"], gi["cu_seqlens"], gi["tile_start"], gi["slot_ids"],
                          gi["cu_cached"], N, 16, 8, wl.block_m)
    dplan = K.decode_plan(gi["cached_lens"], gi["num_decoding"], gi["slot_ids"].shape[0], 16, 8)
    ms_planned = time_graph(lambda: op(plan, dplan))
    return {"us_graph": round(ms * 1e3, 2), "us_graph_planned": round(ms_planned * 1e3, 2),
            "planned": "the step's prefill and decode work lists computed once per step (not "
                       "timed here: 28 layers share them) and read by the launches",
            "rows": N, "decoders": len(wl.decode_ctx),
            "prefill_tokens": sum(L for L, _ in wl.chunks),
            "kernels": "fused_norm_rope_prefill, quantize_kv_prefill, prefill_attention, "
                       "decode_attention_rope (fused_rope_kv_decode + decode_attention)"}


def bench_step(steps, warmup, dev):
    """Config 5: graph replays of the whole decode step and of its attention kernels alone."""
    ds = importlib.import_module("inference-engine_amd.decode_step")
    B = 32
    step = ds.make_decode_step(batch=B, ctx_lo=128, ctx_hi=4096, device=dev, seed=0)
    g_step, _ = step.capture()
    g_attn, _ = step.capture(step.attention_only)

    def t(graph):
        for _ in range(warmup):
            graph.replay()
        settle(graph.replay)
        e0, e1 = _events(2)
        e0.record()
        for _ in range(steps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    ms_step, ms_attn = t(g_step), t(g_attn)
    res = {"tokens_per_s": round(B / (ms_step * 1e-3), 1), "ms_per_step": round(ms_step, 4),
           "attention_ms": round(ms_attn, 4), "attention_share": round(ms_attn / ms_step, 4),
           "batch": B, "layers": step.shape.layers, "ctx_mean": round(
               float(step.cached_lens.float().mean().item()) + 1, 1),
           "fused_layers": step.fused,
           "graph": "torch.cuda.CUDAGraph (hipGraph) of the full step; attention share = replay "
                    "time of the step's attention kernel (decode_attention_rope: "
                    "fused_rope_kv_decode + decode_attention in one launch) captured alone / "
                    "step replay time; fused_layers: both add_rms_norm launches of every layer "
                    "inside the projections (RMSNorm weights folded into qkv and gate_up, "
                    "residual adds in o_proj and down)"}
    del g_step, g_attn, step
    torch.cuda.empty_cache()
    # the reference's layer form (add_rms_norm launches between the projections), same seed
    step = ds.make_decode_step(batch=B, ctx_lo=128, ctx_hi=4096, device=dev, seed=0,
                               fused=False)
    g_ref, _ = step.capture()
    ms_ref = t(g_ref)
    res["reference_form"] = {"tokens_per_s": round(B / (ms_ref * 1e-3), 1),
                             "ms_per_step": round(ms_ref, 4)}
    del g_ref, step
    torch.cuda.empty_cache()
    return res


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return os.uname().machine


def read_traffic():
    """HBM bytes per launch of the decode kernel from the committed rocprofv3 PMC summary."""
    p = REPO / "profiles" / "decode_attention_B64_ctx4096_pmc.md"
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1].strip())
    return None


def line_read_probe(args, ie, W, K, dev, alg_bytes, extra):
    """The attainable read rate on this device: a pure 16-byte read stream (ie_hbm_read_probe)
    over as many bytes as one decode launch reads, past the 256 MB last-level cache, two buffers
    alternating; and torch's own sum over the same bytes."""
    import ctypes
    lib = importlib.import_module("inference-engine_amd._native").cabi()
    probes = [torch.ones(alg_bytes // 4, dtype=torch.float32, device=dev) for _ in range(2)]
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    turn = [0]

    def read_probe():
        t = probes[turn[0]]
        turn[0] ^= 1
        rc = lib.ie_hbm_read_probe(ctypes.c_void_p(t.data_ptr()), ctypes.c_size_t(alg_bytes),
                                   ctypes.c_uint32(0x9E3779B9), ctypes.c_void_p(sink.data_ptr()),
                                   stream)
        assert rc == 0, lib.ie_attn_last_error()
    rp_ms = time_op(read_probe, args.steps, args.warmup)
    ts_ms = time_op(lambda: probes[0].sum(), args.steps, args.warmup)
    extra["read_probe"] = {"bytes": alg_bytes,
                           "stream_us": round(rp_ms * 1e3, 2),
                           "stream_GBps": round(alg_bytes / (rp_ms * 1e-3) / 1e9, 1),
                           "torch_sum_GBps": round(alg_bytes / (ts_ms * 1e-3) / 1e9, 1)}
    log(f"read probe {rp_ms*1e3:.2f} us, torch.sum {ts_ms*1e3:.2f} us")

    # Config 5's decode launch beside the same stream over its bytes: B=32, ctx ~ U[128, 4096)
    # as decode_step draws it; the stream reads four regions in turn (past the 256 MB cache)
    g = torch.Generator().manual_seed(0)
    c5 = torch.randint(128, 4096, (32,), generator=g).tolist()
    c5_wls = [W.decode_workload(c5, seed=s, device=dev) for s in range(2)]
    c5_bytes = c5_wls[0].algorithmic_bytes() // 16 * 16
    assert 2 * c5_bytes <= alg_bytes
    regions = [(t, off) for t in probes for off in (0, alg_bytes // 2 // 16 * 16)]

    def read_probe_c5():
        t, off = regions[turn[0] % 4]
        turn[0] += 1
        rc = lib.ie_hbm_read_probe(ctypes.c_void_p(t.data_ptr() + off), ctypes.c_size_t(c5_bytes),
                                   ctypes.c_uint32(0x9E3779B9), ctypes.c_void_p(sink.data_ptr()),
                                   stream)
        assert rc == 0, lib.ie_attn_last_error()
    rp5_ms = time_op(read_probe_c5, args.steps, args.warmup)
    dec5_ms = time_decode(ie, c5_wls, args.steps, args.warmup)
    extra["read_probe"]["config5"] = {
        "bytes": c5_bytes, "stream_us": round(rp5_ms * 1e3, 2),
        "decode_us": round(dec5_ms * 1e3, 2),
        "decode_GBps": round(c5_bytes / (dec5_ms * 1e-3) / 1e9, 1),
        "decode_over_stream": round(rp5_ms / dec5_ms, 3)}
    log(f"config 5 bytes {c5_bytes / 1e6:.1f} MB: read probe {rp5_ms*1e3:.2f} us, "
        f"decode {dec5_ms*1e3:.2f} us")


def line_kv_write(args, ie, W, K, dev, alg_bytes, extra):
    """Config 4's KV quantize-on-write (1,024 new tokens), and a long step: a first chunk of 8192
    tokens (with its calibration) and 4096 new tokens after 4096 cached, where the write is
    bandwidth-bound rather than latency-bound."""
    mw = W.mixed_to(W.config4(seed=0), dev)
    gi = mw.inputs
    kv_op = lambda: K.quantize_kv_prefill(mw.k, mw.v, gi["cu_seqlens"], gi["slot_ids"],
                                          gi["cached_lens"], gi["num_decoding"], mw.cache)
    kv_ms = time_op(kv_op, args.steps, args.warmup)
    kv_gms = time_graph(kv_op)
    n_new = sum(L for L, _ in mw.chunks)
    kv_bytes = n_new * 8 * (128 * 2 * 2 + 128 * 2 + 8)
    extra["kv_write_config4"] = {"us": round(kv_ms * 1e3, 3),
                                 "GBps": round(kv_bytes / (kv_ms * 1e-3) / 1e9, 1),
                                 "us_graph": round(kv_gms * 1e3, 3), "bytes": kv_bytes}
    log(f"kv write config4 {kv_ms*1e3:.2f} us")
    lw = W.mixed_to(W.mixed_workload([], [(8192, 0), (4096, 4096)], seed=1, block_m=128,
                                     max_len=8192), dev)
    li = lw.inputs
    kvl_op = lambda: K.quantize_kv_prefill(lw.k, lw.v, li["cu_seqlens"], li["slot_ids"],
                                           li["cached_lens"], li["num_decoding"], lw.cache)
    kvl_ms = time_op(kvl_op, args.steps, args.warmup)
    kvl_bytes = (8192 + 4096) * 8 * (128 * 2 * 2 + 128 * 2 + 8)
    extra["kv_write_long"] = {"tokens": 8192 + 4096, "us": round(kvl_ms * 1e3, 3),
                              "GBps": round(kvl_bytes / (kvl_ms * 1e-3) / 1e9, 1),
                              "bytes": kvl_bytes}
    log(f"kv write long {kvl_ms*1e3:.2f} us")


def line_prefill_config4(args, ie, W, K, dev, alg_bytes, extra):
    """Config 4's chunked-prefill attention (one launch; split pieces merge in it),
    causal-exact flops."""
    mw = W.mixed_to(W.config4(seed=0), dev)
    gi = mw.inputs
    flops = W.prefill_flops(mw.chunks)
    pf_op = lambda: K.prefill_attention(
        mw.q, mw.k, mw.v, gi["seq_ids"], gi["cu_seqlens"], gi["tile_start"], mw.cache,
        gi["slot_ids"], gi["cu_cached"], mw.block_m)
    pf_ms = time_op(pf_op, args.steps, args.warmup)
    pf_gms = time_graph(pf_op)
    # the work list computed once per step (every layer of the step reuses it)
    plan_op = lambda: K.prefill_plan(gi["seq_ids"], gi["cu_seqlens"], gi["tile_start"],
                                     gi["slot_ids"], gi["cu_cached"], mw.q.shape[0],
                                     mw.q.shape[1], mw.cache.k.shape[1], mw.block_m)
    plan = plan_op()
    pp_op = lambda: K.prefill_attention(
        mw.q, mw.k, mw.v, gi["seq_ids"], gi["cu_seqlens"], gi["tile_start"], mw.cache,
        gi["slot_ids"], gi["cu_cached"], mw.block_m, plan)
    pp_ms = time_op(pp_op, args.steps, args.warmup)
    pp_gms = time_graph(pp_op)
    plan_gms = time_graph(plan_op)
    tf = flops / (pf_ms * 1e-3) / 1e12
    frac = lambda ms: round(flops / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)
    extra["prefill_config4"] = {"us": round(pf_ms * 1e3, 3), "TFLOPs": round(tf, 1),
                                "mfma_frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
                                "us_graph": round(pf_gms * 1e3, 3),
                                "mfma_frac_graph": frac(pf_gms),
                                "planned": {"us": round(pp_ms * 1e3, 3), "mfma_frac": frac(pp_ms),
                                            "us_graph": round(pp_gms * 1e3, 3),
                                            "mfma_frac_graph": frac(pp_gms),
                                            "plan_us_graph": round(plan_gms * 1e3, 3),
                                            "note": "prefill_plan once per step, its rows read "
                                                    "by every layer's launch"},
                                "flops": flops}
    log(f"prefill config4 {pf_ms*1e3:.2f} us {tf:.1f} TFLOP/s; planned {pp_ms*1e3:.2f} us")


def line_prefill_long(args, ie, W, K, dev, alg_bytes, extra):
    """Long prefills, where the tile loop rather than the per-launch latency sets the time:
    4 x 2048 new tokens after 2048 cached, 4 x 1024 new after 7168 cached, and 4 x 512 new
    after 8192 cached (few query rows over long prefixes: the pairs are split into pieces that
    cross from the prefix into the chunk)."""
    longs = {}
    for name, chunks, max_len in (("4x2048_after_2048", [(2048, 2048)] * 4, 4096),
                                  ("4x1024_after_7168", [(1024, 7168)] * 4, 8192),
                                  ("4x512_after_8192", [(512, 8192)] * 4, 8704)):
        pw = W.mixed_to(W.mixed_workload([], chunks, seed=2, block_m=128, max_len=max_len), dev)
        pi = pw.inputs
        op = lambda: K.prefill_attention(
            pw.q, pw.k, pw.v, pi["seq_ids"], pi["cu_seqlens"], pi["tile_start"], pw.cache,
            pi["slot_ids"], pi["cu_cached"], pw.block_m)
        ms = time_op(op, args.steps, args.warmup)
        fl = W.prefill_flops(pw.chunks)
        tf = fl / (ms * 1e-3) / 1e12
        longs[name] = {"us": round(ms * 1e3, 2), "TFLOPs": round(tf, 1),
                       "mfma_frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4), "flops": fl}
        log(f"prefill {name} {ms*1e3:.2f} us {tf:.1f} TFLOP/s")
        del pw, pi, op
    extra["prefill_long"] = longs


def line_norm_rope(args, ie, W, K, dev, alg_bytes, extra):
    """Config 4: prefill q/k RMSNorm + RoPE of the 1,024 packed prefill tokens."""
    extra["norm_rope_prefill_config4"] = bench_norm_rope(K, args.norm_rope_tokens, args.steps,
                                                         args.warmup, dev)
    log(f"norm rope prefill config4 {extra['norm_rope_prefill_config4']}")


def line_sample(args, ie, W, K, dev, alg_bytes, extra):
    """Config 5's sampler: B = 32 rows of the 151,936-entry vocabulary."""
    extra["sample_config5"] = bench_sample(K, 32, 151_936, args.steps, args.warmup, dev)
    log(f"sample config5 {extra['sample_config5']}")


def line_linear(args, ie, W, K, dev, alg_bytes, extra):
    """Config 5's projections at 32 rows."""
    extra["linear_config5"] = bench_linear(K, 32, dev)
    log(f"linear config5 {extra['linear_config5']}")


def line_launch_floor(args, ie, W, K, dev, alg_bytes, extra):
    """What one small kernel costs inside a hipGraph: 56 dependent add_rms_norm calls at config
    5's 32 x 2048 (a step's worth) against 56 one-element torch adds (a launch that does no
    work), each captured in one graph and replayed. A profiler's kernel trace inflates such
    kernels inside graph replays to about 4.5 us each, torch's own included."""
    res = torch.randn(32, 2048, device=dev).bfloat16()
    dl = torch.randn(32, 2048, device=dev).bfloat16()
    w = torch.randn(2048, device=dev).bfloat16()
    tiny = torch.zeros(1, device=dev)
    state = {"r": res}

    def rms():
        state["r"], _ = K.add_rms_norm(state["r"], dl, w, 1e-6)

    rms_ms = time_graph(rms, calls=56, reps=20)
    add_ms = time_graph(lambda: tiny.add_(1.0), calls=56, reps=20)
    extra["graph_launch_floor"] = {"add_rms_norm_us": round(rms_ms * 1e3, 2),
                                   "torch_add_1elem_us": round(add_ms * 1e3, 2),
                                   "calls_per_graph": 56, "rows": 32, "dim": 2048}
    log(f"graph launch floor {extra['graph_launch_floor']}")


def line_mixed_step(args, ie, W, K, dev, alg_bytes, extra):
    extra["mixed_step_config4"] = bench_mixed_step(W, dev)
    log(f"mixed step config4 {extra['mixed_step_config4']}")


def line_step(args, ie, W, K, dev, alg_bytes, extra):
    log("config 5: Qwen3-1.7B-shaped decode step (hipGraph)")
    extra["decode_step_config5"] = bench_step(max(10, args.steps // 2), 3, dev)
    log(f"config5 {extra['decode_step_config5']}")


def line_sweep(args, ie, W, K, dev, alg_bytes, extra):
    """The config-3 shape sweep: whole decode_attention steps, two rotated cache sets."""
    sweep = {}
    for b in (16, 64, 256):
        for c in (1024, 4096):
            ws = [W.decode_workload([c] * b, seed=s, device=dev) for s in range(2)]
            sm = time_decode(ie, ws, 20, 5)
            by = ws[0].algorithmic_bytes()
            sweep[f"B{b}_ctx{c}"] = {"us": round(sm * 1e3, 2),
                                     "GBps": round(by / (sm * 1e-3) / 1e9, 1)}
            log(f"sweep B={b} ctx={c}: {sm*1e3:.2f} us")
            del ws
            torch.cuda.empty_cache()
    extra["decode_sweep"] = sweep


# the lines beside the headline, in the order they run (--lines picks a subset)
LINES = {"read_probe": line_read_probe, "kv_write": line_kv_write,
         "prefill_config4": line_prefill_config4, "prefill_long": line_prefill_long,
         "norm_rope": line_norm_rope, "sample": line_sample, "linear": line_linear,
         "launch_floor": line_launch_floor, "mixed_step": line_mixed_step, "step": line_step,
         "sweep": line_sweep}
DEFAULT_LINES = [n for n in LINES if n != "sweep"]


def extras(args, ie, W, K, dev, alg_bytes) -> dict:
    """Every line beside the headline that --lines selects; a line that fails reports its error
    under its own key instead of its numbers."""
    extra = {}
    for name in args.lines:
        torch.cuda.empty_cache()
        try:
            LINES[name](args, ie, W, K, dev, alg_bytes, extra)
        except Exception as e:  # reported, never silently replaced
            extra[f"{name}_error"] = str(e).splitlines()[0][:200]
    return extra


def prefill_phase_stamps(W, dev, warmup, planned=False):
    """Config 4's prefill attention through the C ABI of the phase-stamp build
    (inference-engine_amd/lib/stamps/libie_attn.so: the same kernel with a 100 MHz clock read
    by thread 0 of every workgroup at each phase boundary). Per call: the time from the first
    workgroup's start to each workgroup's phase boundaries; medians over five calls after
    `warmup` calls that bring the clocks up. planned: the work list is computed once
    (ie_prefill_attention_plan) and every call reads it (ie_prefill_attention_planned)."""
    import ctypes
    import numpy as np
    path = REPO / "inference-engine_amd" / "lib" / "stamps" / "libie_attn.so"
    if not path.exists():
        raise SystemExit(f"{path} is missing: run python inference-engine_amd/build.py --stamps")
    lib = ctypes.CDLL(str(path))
    lib.ie_prefill_attention_workspace_size.restype = ctypes.c_size_t
    lib.ie_attn_last_error.restype = ctypes.c_char_p
    NT = importlib.import_module("inference-engine_amd._native")
    mw = W.mixed_to(W.config4(seed=0), dev)
    gi = mw.inputs
    N, nt = mw.q.shape[0], gi["tile_start"].shape[0]
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    desc = NT.KVCacheDesc.of(mw.cache)
    wsb = lib.ie_prefill_attention_workspace_size(nt, mw.block_m, 8)
    ws = torch.zeros(int(wsb), dtype=torch.uint8, device=dev)
    out = torch.empty_like(mw.q)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    i64, i32 = ctypes.c_int64, ctypes.c_int32
    grid = lib.ie_prefill_attention_grid(i32(nt), i32(mw.block_m), i32(16), i32(8))
    rows = torch.empty(grid, 16, dtype=torch.int32, device=dev)
    if planned:
        assert lib.ie_prefill_attention_plan(
            p(gi["seq_ids"]), p(gi["cu_seqlens"]), p(gi["tile_start"]), i32(nt),
            i32(mw.block_m), i64(N), i32(16), i32(8), p(gi["slot_ids"]), p(gi["cu_cached"]),
            i32(gi["slot_ids"].shape[0]), p(rows), stream) == 0, lib.ie_attn_last_error()

    def run():
        head = (p(mw.q), i64(mw.q.stride(0)), i64(mw.q.stride(1)), p(mw.k), i64(mw.k.stride(0)),
                i64(mw.k.stride(1)), p(mw.v), i64(mw.v.stride(0)), i64(mw.v.stride(1)), i64(N),
                i32(16), p(gi["seq_ids"]), p(gi["cu_seqlens"]), p(gi["tile_start"]), i32(nt),
                i32(mw.block_m), ctypes.byref(desc), p(gi["slot_ids"]), p(gi["cu_cached"]),
                i32(gi["slot_ids"].shape[0]))
        tail = (p(out), i64(out.stride(0)), i64(out.stride(1)), p(ws), ctypes.c_size_t(wsb),
                stream)
        if planned:
            rc = lib.ie_prefill_attention_planned(*head, p(rows), i64(grid), *tail)
        else:
            rc = lib.ie_prefill_attention(*head, *tail)
        assert rc == 0, lib.ie_attn_last_error()

    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    nwg, words = 4096, 9
    buf = (ctypes.c_ulonglong * (nwg * words))()
    assert lib.ie_prefill_phase_stamps_copy(buf, ctypes.c_size_t(nwg * words), 1) == 0
    calls = []
    for _ in range(5):
        for _ in range(20):  # the clocks stay up; these calls' stamps are cleared below
            run()
        torch.cuda.synchronize()
        assert lib.ie_prefill_phase_stamps_copy(buf, ctypes.c_size_t(nwg * words), 1) == 0
        run()
        torch.cuda.synchronize()
        assert lib.ie_prefill_phase_stamps_copy(buf, ctypes.c_size_t(nwg * words), 1) == 0
        t = np.array(buf, dtype=np.int64).reshape(nwg, words)
        t = t[t[:, 0] > 0]
        calls.append(t)
    names = ["start", "work_list", "first_scores", "tiles_done", "partial_written",
             "wait_over", "share_merged", "end"]
    res = {}
    for i, nm in enumerate(names):
        vals = []
        for t in calls:
            base = t[:, 0].min()
            col = t[:, i]
            vals.append((col[col > 0] - base) * 0.01)  # us
        v = np.concatenate(vals)
        if len(v):
            res[nm] = {"p50_us": round(float(np.median(v)), 2),
                       "p90_us": round(float(np.percentile(v, 90)), 2),
                       "max_us": round(float(v.max()), 2), "workgroups": int(len(v) // 5)}
    steps = {}
    for a, b in ((0, 1), (1, 2), (2, 3), (3, 4), (4, 5), (5, 6), (6, 7), (3, 7)):
        d = np.concatenate([(t[:, b] - t[:, a])[(t[:, a] > 0) & (t[:, b] > 0)] * 0.01
                            for t in calls])
        if len(d):
            steps[f"{names[a]}->{names[b]}"] = {"p50_us": round(float(np.median(d)), 2),
                                                "p90_us": round(float(np.percentile(d, 90)), 2)}
    pieces = calls[0][:, 8]
    # workgroup w runs on XCD w mod 8: start and end of the workgroups with work, per XCD
    by_xcd = {}
    for x in range(8):
        st, en = [], []
        for t in calls:
            ids = np.arange(len(t))
            sel = (ids % 8 == x) & (t[:, 8] > 0) & (t[:, 7] > 0)
            st.append((t[sel, 0] - t[:, 0].min()) * 0.01)
            en.append((t[sel, 7] - t[:, 0].min()) * 0.01)
        st, en = np.concatenate(st), np.concatenate(en)
        if len(st):
            by_xcd[str(x)] = {"start_p50_us": round(float(np.median(st)), 2),
                              "end_p50_us": round(float(np.median(en)), 2),
                              "end_max_us": round(float(en.max()), 2)}
    return {"workload": "prefill_attention config 4 (phase-stamp build" +
                        (", precomputed work list)" if planned else ")"),
            "call_us_last_end": round(float(np.median([(t[:, 7].max() - t[:, 0].min()) * 0.01
                                                       for t in calls])), 2),
            "workgroups_with_work": int((pieces > 0).sum()),
            "split_pieces": int((pieces > 1).sum()), "phases": res, "steps": steps,
            "by_xcd": by_xcd}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # the warm-up also brings the device's clocks up from idle: 300 decode steps (~27 ms) do;
    # 10 measured 3-5 % slower on the same box
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--rotate", type=int, default=2, help="distinct cache sets cycled per step")
    ap.add_argument("--settle-ms", type=float, default=150.0,
                    help="minimum warm-up wall time of each line beside the headline, after its "
                         "--warmup calls (untimed; lets the clocks come up, see settle())")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="minimum CPU-baseline decode work (whole batch, repeated); the config-4 "
                         "KV write and prefill baselines run a third of it each")
    ap.add_argument("--no-step", action="store_true", help="skip the config-5 decode step")
    ap.add_argument("--lines", default=",".join(DEFAULT_LINES),
                    help=f"comma-separated lines beside the headline, of {','.join(LINES)} "
                         "(default: all but sweep)")
    ap.add_argument("--norm-rope-tokens", type=int, default=1024,
                    help="packed tokens of the prefill norm/rope line (config 4: 1024)")
    ap.add_argument("--sweep", action="store_true", help="also time the config-3 shape sweep")
    ap.add_argument("--headline-only", action="store_true",
                    help="only the headline decode timing (for kernel traces and PMC passes: "
                         "every decode launch of the run is then a headline launch)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="first run a plain device copy of MIB MiB 3 times (PMC calibration)")
    ap.add_argument("--prefill-stamps", nargs="?", const="self", choices=["self", "planned"],
                    help="instead of the bench line: config 4's prefill attention on the "
                         "phase-stamp build (python inference-engine_amd/build.py --stamps), "
                         "per-phase medians of its workgroups as one JSON line; 'planned': "
                         "the launch that reads a precomputed work list")
    args = ap.parse_args()
    global SETTLE_S
    SETTLE_S = args.settle_ms * 1e-3
    args.lines = [x for x in args.lines.split(",") if x]
    bad = [x for x in args.lines if x not in LINES]
    if bad:
        ap.error(f"unknown lines {bad}; known: {list(LINES)}")
    if args.no_step and "step" in args.lines:
        args.lines.remove("step")
    if args.sweep and "sweep" not in args.lines:
        args.lines.append("sweep")

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(decode attention shards by sequence or KV head without exchange); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    ie = importlib.import_module("inference-engine_amd")
    W = importlib.import_module("inference-engine_amd.workloads")
    K = ie.kernels
    dev = "cuda:0"
    torch.cuda.set_device(0)

    if args.prefill_stamps:
        print(json.dumps(prefill_phase_stamps(W, dev, args.warmup,
                                              args.prefill_stamps == "planned")), flush=True)
        return

    if args.copy_probe:
        n = args.copy_probe << 20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: 3 x {n} bytes read + written")
        del src, dst

    ctx = [args.ctx] * args.batch
    log(f"building {args.rotate} cache sets B={args.batch} ctx={args.ctx}")
    wls = [W.decode_workload(ctx, seed=s, device=dev) for s in range(args.rotate)]
    torch.cuda.synchronize()
    alg_bytes = wls[0].algorithmic_bytes()
    log("timing decode attention")
    step_ms = time_decode(ie, wls, args.steps, args.warmup)
    gbs = alg_bytes / (step_ms * 1e-3) / 1e9
    log(f"decode step (one launch of decode_attention_kernel) {step_ms*1e3:.2f} us ({gbs:.0f} GB/s)")

    extra = {}
    if args.headline_only:
        args.no_cpu = True
    else:
        extra.update(extras(args, ie, W, K, dev, alg_bytes))

    cpu = None
    if not args.no_cpu:
        log(f"cpu baseline (PyTorch on {cpu_threads()} host threads)")
        cpu = cpu_baselines(wls[0], alg_bytes, W, args.cpu_seconds)
        log(f"cpu baseline {cpu}")
    traffic = read_traffic()
    line = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "us_per_layer": round(step_ms * 1e3, 2),
        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "decode_attention B=64 ctx=4096 (BASELINE config 3 headline)",
                   "batch": args.batch, "ctx": args.ctx, "q_heads": 16, "kv_heads": 8,
                   "head_dim": 128, "rotated_cache_sets": args.rotate,
                   "algorithmic_bytes": alg_bytes},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "kernel": "decode_attention_kernel",
                     "kernel_us": round(step_ms * 1e3, 2),
                     "kernel_us_from": "back-to-back launches between two HIP events on the "
                                       "launch stream (the op is this one kernel)"},
        "cpu_baseline": cpu,
        **extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
