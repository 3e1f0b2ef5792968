"""Writes the golden fixtures of tests/golden/*.npz from the numpy oracle on seeded inputs.

    python tests/golden/make_golden.py [name ...]     # all fixtures, or the named ones

The reference ships no test vectors, so these fixtures are this build's own pins: the CPU tests
check that the oracle still reproduces them exactly (a regression guard on the restatement,
which is itself pinned by closed forms and float64 checks), and the GPU tests run the HIP path
on the same inputs. Every fixture is small (well under 1 MB) and holds inputs as raw bits
(bf16 as uint16) next to the expected outputs.
"""

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO))

from oracle import attention as oat  # noqa: E402
from oracle import kv_cache as okv  # noqa: E402
from oracle.numerics import bf16_bits, bits_to_f32  # noqa: E402

W = __import__("importlib").import_module("inference-engine_amd.workloads")

SCALE = 128 ** -0.5


def _bf16(t: torch.Tensor) -> np.ndarray:
    return t.float().numpy()


def _arrays(c) -> okv.CacheArrays:
    return okv.CacheArrays(*(t.numpy().copy() for t in
                             (c.k, c.v, c.k_scale, c.v_scale, c.k_calibration)))


def _copy(a: okv.CacheArrays) -> okv.CacheArrays:
    return okv.CacheArrays(a.k.copy(), a.v.copy(), a.k_scale.copy(), a.v_scale.copy(),
                           a.k_calibration.copy())


def _cache_dict(prefix, c):
    return {f"{prefix}_k": c.k, f"{prefix}_v": c.v, f"{prefix}_k_scale": c.k_scale,
            f"{prefix}_v_scale": c.v_scale, f"{prefix}_k_cal": c.k_calibration}


def quant_rows():
    """Known-answer rows plus seeded random bf16 rows through quantize_rows (per-row int8 +
    scale): all zero, one-hot, exact .5 ties, values at the clamp, tiny and huge magnitudes."""
    rows = np.zeros((16, 128), np.float32)
    rows[1, 5] = 3.0  # one-hot -> +127 at 5
    rows[2, 0] = -1e-3
    rows[3, :] = np.linspace(-2.0, 2.0, 128, dtype=np.float32)
    rows[4, :4] = [127.0, 63.5, -0.5, 1.5]  # s = 1: exact ties at 63.5, -0.5, 1.5
    rows[5, :] = 1e-8  # below the 1e-6 scale floor
    rows[6, :] = 3.0e4
    rows[6, 1] = -3.0e4
    g = torch.Generator().manual_seed(11)
    rows[7:] = torch.randn(9, 128, generator=g).bfloat16().float().numpy() * np.float32(
        [0.01, 0.1, 1, 3, 10, 100, 1000, 1e-3, 7])[:, None]
    rows = bits_to_f32(bf16_bits(rows))  # bf16-representable, as every cache write input is
    q, s = okv.quantize_rows(rows)
    return {"rows": rows, "q": q, "s": s}


def prefill_write():
    """quantize_kv_prefill on a small mixed step: 2 decoders (untouched), a first chunk (the
    calibration is computed and stored) and a chunk after 9 cached tokens (stored calibration)."""
    wl = W.mixed_workload([5, 9], [(24, 0), (7, 9), (0, 0)], seed=12, block_m=32, max_len=64)
    ins = {n: t.numpy() for n, t in wl.inputs.items()}
    before = _arrays(wl.cache)
    after = _copy(before)
    okv.quantize_kv_prefill(_bf16(wl.k), _bf16(wl.v), ins["cu_seqlens"], ins["slot_ids"],
                            ins["cached_lens"], int(ins["num_decoding"][0]), after)
    out = {"k_bits": bf16_bits(_bf16(wl.k)), "v_bits": bf16_bits(_bf16(wl.v.contiguous())),
           **{f"in_{n}": a for n, a in ins.items()}}
    for name in ("k", "v", "k_scale", "v_scale", "k_calibration"):
        out[f"before_{name}"] = getattr(before, name)
        out[f"after_{name}"] = getattr(after, name)
    return out


def rope_kv_decode():
    """fused_rope_kv_decode for 3 sequences (norm + RoPE + q x calibration + K/V write)."""
    g = torch.Generator().manual_seed(13)
    B, pool, L = 3, 4, 16
    qkv = torch.randn(B, 32 * 128, generator=g).bfloat16()
    qw = (1 + 0.1 * torch.randn(128, generator=g)).bfloat16()
    kw = (1 + 0.1 * torch.randn(128, generator=g)).bfloat16()
    cached = np.array([0, 7, 15], np.int32)
    slots = np.array([2, 0, 3], np.int32)
    inv = 1e6 ** (-torch.arange(0, 128, 2, dtype=torch.float32) / 128)
    ang = torch.from_numpy(cached).float()[:, None, None] * inv[None, None, :]
    cos, sin = ang.cos().bfloat16(), ang.sin().bfloat16()
    cache = W.empty_cache(pool, L)
    cache.k_calibration.copy_(0.5 + torch.rand(cache.k_calibration.shape, generator=g))
    arr = _arrays(cache)
    q = _bf16(qkv[:, :2048].view(B, 16, 128))
    k = _bf16(qkv[:, 2048:3072].view(B, 8, 128))
    v = _bf16(qkv[:, 3072:].view(B, 8, 128))
    q_out = okv.fused_rope_kv_decode(q, k, v, _bf16(qw), _bf16(kw), _bf16(cos), _bf16(sin),
                                     slots, arr, cached, B, 1e-6)
    return {"qkv_bits": bf16_bits(_bf16(qkv)), "qw_bits": bf16_bits(_bf16(qw)),
            "kw_bits": bf16_bits(_bf16(kw)), "cos_bits": bf16_bits(_bf16(cos)),
            "sin_bits": bf16_bits(_bf16(sin)), "cached_lens": cached, "slot_ids": slots,
            "cal": cache.k_calibration.numpy(), "q_out_bits": bf16_bits(q_out),
            "after_k": arr.k, "after_v": arr.v, "after_k_scale": arr.k_scale,
            "after_v_scale": arr.v_scale}


def norm_rope_prefill():
    """fused_norm_rope_prefill for 19 packed prefill tokens of two chunks (positions 0..10 and
    500..507): q/k are strided views of one fused qkv row, RoPE tables as the engine builds
    them (architecture.py:343-354: inv_freq = 1e6^(-2i/128), angle = position * inv_freq)."""
    g = torch.Generator().manual_seed(16)
    N = 19
    qkv = (2 * torch.randn(N, 32 * 128, generator=g)).bfloat16()
    qw = (1 + 0.1 * torch.randn(128, generator=g)).bfloat16()
    kw = (1 + 0.1 * torch.randn(128, generator=g)).bfloat16()
    pos = torch.cat([torch.arange(0, 11), torch.arange(500, 508)]).float()
    inv = 1e6 ** (-torch.arange(0, 128, 2, dtype=torch.float32) / 128)
    ang = pos[:, None, None] * inv[None, None, :]
    cos, sin = ang.cos().bfloat16(), ang.sin().bfloat16()
    q = _bf16(qkv[:, :2048].view(N, 16, 128))
    k = _bf16(qkv[:, 2048:3072].view(N, 8, 128))
    q_out, k_out = okv.fused_norm_rope_prefill(q, k, _bf16(qw), _bf16(kw), _bf16(cos),
                                               _bf16(sin), 1e-6)
    return {"qkv_bits": bf16_bits(_bf16(qkv)), "qw_bits": bf16_bits(_bf16(qw)),
            "kw_bits": bf16_bits(_bf16(kw)), "cos_bits": bf16_bits(_bf16(cos)),
            "sin_bits": bf16_bits(_bf16(sin)), "q_out_bits": bf16_bits(q_out),
            "k_out_bits": bf16_bits(k_out)}


def decode_config1():
    """BASELINE config 1 (B=1, ctx=128) decode attention: inputs and the oracle's output."""
    wl = W.decode_workload([128], seed=14)
    c = wl.cache
    ref = oat.decode_attention(_bf16(wl.q), _arrays(c), wl.cached_lens.numpy(),
                               wl.slot_ids.numpy(), 1, SCALE)
    return {"q_bits": bf16_bits(_bf16(wl.q)), **_cache_dict("cache", c),
            "cached_lens": wl.cached_lens.numpy(), "slot_ids": wl.slot_ids.numpy(),
            "out": ref.astype(np.float32)}


def prefill_small():
    """Chunked-prefill attention: 2 decoders, a 20-row chunk after a 40-token cached prefix and
    an 11-row first chunk, block_m 16 (tiles cross no entry)."""
    wl = W.mixed_workload([6, 3], [(20, 40), (11, 0)], seed=15, block_m=16, max_len=128)
    ins = {n: t.numpy() for n, t in wl.inputs.items()}
    c = wl.cache
    arr = _arrays(c)
    kp, vp = okv.dequantize_kv_prefix(arr, ins["cu_cached"], ins["slot_ids"])
    ref = oat.prefill_attention(_bf16(wl.q), _bf16(wl.k), _bf16(wl.v), ins["cu_seqlens"],
                                ins["tile_start"], wl.block_m, kp, vp, ins["cu_cached"])
    return {"q_bits": bf16_bits(_bf16(wl.q)), "k_bits": bf16_bits(_bf16(wl.k)),
            "v_bits": bf16_bits(_bf16(wl.v.contiguous())), **_cache_dict("cache", c),
            **{f"in_{n}": a for n, a in ins.items()}, "block_m": np.int32(wl.block_m),
            "out": ref.astype(np.float32)}


FIXTURES = {
    "quant_rows": quant_rows,
    "prefill_write": prefill_write,
    "rope_kv_decode": rope_kv_decode,
    "norm_rope_prefill": norm_rope_prefill,
    "decode_config1": decode_config1,
    "prefill_small": prefill_small,
}


def _np(d):
    return {k: (v.numpy() if isinstance(v, torch.Tensor) else np.asarray(v)) for k, v in d.items()}


def main():
    names = sys.argv[1:] or list(FIXTURES)
    for name in names:
        fn = FIXTURES[name]
        path = HERE / f"{name}.npz"
        np.savez_compressed(path, **_np(fn()))
        print(f"wrote {path.relative_to(REPO)} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
