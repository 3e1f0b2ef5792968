"""Seeded synthetic inputs for the benchmark configurations (shapes of BASELINE configs 1-4).

Everything is generated from a seeded torch.Generator, as bf16 ~ N(0, 1) sources quantized into
the int8 cache with the quantize-on-write formula (per (token, kv head) scale = max|x|/127,
cache calibration 1 unless stated). "ctx" counts the tokens a decoding sequence attends to, so
cached_lens = ctx - 1 and columns [0, ctx) of its cache row are filled.

These helpers only build input data; every op measured or tested runs through `kernels`.
"""

import math
from dataclasses import dataclass

import torch

from .kernels import LayerKVCache
from .step_inputs import fill_inputs

HQ, HKV, D = 16, 8, 128


def quantize_rows(x: torch.Tensor):
    """Symmetric int8 per row of a float32 tensor: s = max(max|x|, 1e-6)/127, q = round(x/s)."""
    x = x.float()
    s = x.abs().amax(dim=-1).clamp_min(1e-6) / 127.0
    q = torch.round(x / s.unsqueeze(-1)).clamp_(-127, 127).to(torch.int8)
    return q, s


def randn_bf16(shape, gen, device="cpu") -> torch.Tensor:
    return torch.randn(shape, generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)


def empty_cache(pool, max_len, device="cpu", hkv: int = HKV) -> LayerKVCache:
    return LayerKVCache(
        k=torch.zeros(pool, hkv, max_len, D, dtype=torch.int8, device=device),
        v=torch.zeros(pool, hkv, max_len, D, dtype=torch.int8, device=device),
        k_scale=torch.zeros(pool, hkv, max_len, dtype=torch.float32, device=device),
        v_scale=torch.zeros(pool, hkv, max_len, dtype=torch.float32, device=device),
        k_calibration=torch.ones(pool, hkv, 1, D, dtype=torch.float32, device=device),
    )


def fill_rows(cache: LayerKVCache, slot: int, n: int, gen, calibrate=False,
              v_mult: float = 1.0) -> None:
    """Columns [0, n) of cache row `slot` from bf16 N(0,1) K/V (V times `v_mult`, rounded to
    bf16); optional per-channel calibration max(1e-3, max_t |k|) (the first-chunk rule)
    applied to K before quantizing."""
    if n <= 0:
        return
    dev = cache.k.device
    hkv = cache.k.shape[1]
    k = randn_bf16((hkv, n, D), gen, dev).float()
    v = randn_bf16((hkv, n, D), gen, dev).float()
    if v_mult != 1.0:
        v = (v * v_mult).to(torch.bfloat16).float()
    if calibrate:
        cal = k.abs().amax(dim=1).clamp_min(1e-3)  # [HKV, D]
        cache.k_calibration[slot, :, 0] = cal
        k = k / cal[:, None, :]
    kq, ks = quantize_rows(k)
    vq, vs = quantize_rows(v)
    cache.k[slot, :, :n] = kq
    cache.v[slot, :, :n] = vq
    cache.k_scale[slot, :, :n] = ks
    cache.v_scale[slot, :, :n] = vs


@dataclass
class DecodeWorkload:
    q: torch.Tensor  # bf16 [B, HQ, D]
    cache: LayerKVCache
    cached_lens: torch.Tensor  # int32 [B]
    slot_ids: torch.Tensor  # int32 [B]
    num_decoding: torch.Tensor  # int32 [1]
    ctx: list

    def to(self, device) -> "DecodeWorkload":
        c = self.cache
        return DecodeWorkload(
            self.q.to(device),
            LayerKVCache(*(t.to(device) for t in (c.k, c.v, c.k_scale, c.v_scale,
                                                    c.k_calibration))),
            self.cached_lens.to(device), self.slot_ids.to(device), self.num_decoding.to(device),
            list(self.ctx))

    def algorithmic_bytes(self) -> int:
        """int8 K+V rows and fp32 scales read, bf16 q read and out written."""
        hq, hkv = self.q.shape[1], self.cache.k.shape[1]
        return sum(self.ctx) * hkv * (2 * D + 2 * 4) + len(self.ctx) * hq * D * 2 * 2


def decode_ctx_lens(config: str, seed: int = 0) -> list:
    """Context lengths of BASELINE decode configs: '1', '2', or '3:<B>:<ctx>'."""
    if config == "1":
        return [128]
    if config == "2":
        g = torch.Generator().manual_seed(seed)
        return torch.randint(512, 1025, (8,), generator=g).tolist()
    if config.startswith("3:"):
        _, b, c = config.split(":")
        return [int(c)] * int(b)
    raise ValueError(config)


def decode_workload(ctx: list, seed: int = 0, device="cpu", max_len=None, pool=None,
                    num_decoding=None, v_mult: float = 1.0,
                    sink_alpha: float = 0.0, hq: int = HQ, hkv: int = HKV) -> DecodeWorkload:
    """Decode batch with the given per-sequence contexts; slots are a seeded permutation.

    v_mult scales the V source (the V scales scale with it). sink_alpha > 0 makes token 0 of
    every sequence an attention sink for the first query head of each KV head: its K is
    sink_alpha * q of that head (quantized like every row), so that token's score stands
    sink_alpha * |q|^2 / sqrt(D) above the N(0, 1) scores of the other tokens. hq, hkv: query
    and KV heads (default Qwen3-1.7B's 16 and 8)."""
    B = len(ctx)
    gen = torch.Generator(device=device).manual_seed(seed)
    max_len = max_len or int(math.ceil(max(ctx) / 64) * 64)
    pool = pool or B + 1
    q = randn_bf16((B, hq, D), gen, device)
    perm = torch.randperm(pool, generator=torch.Generator().manual_seed(seed + 1))[:B]
    cache = empty_cache(pool, max_len, device, hkv)
    for b in range(B):
        fill_rows(cache, int(perm[b]), ctx[b], gen, v_mult=v_mult)
        if sink_alpha:
            slot = int(perm[b])
            k0 = (q[b, 0::hq // hkv].float() * sink_alpha).to(torch.bfloat16).float()  # [hkv, D]
            kq, ks = quantize_rows(k0)
            cache.k[slot, :, 0] = kq
            cache.k_scale[slot, :, 0] = ks
    nd = B if num_decoding is None else num_decoding
    return DecodeWorkload(q, cache, torch.tensor([c - 1 for c in ctx], dtype=torch.int32,
                                                 device=device),
                          perm.to(torch.int32).to(device),
                          torch.tensor([nd], dtype=torch.int32, device=device), list(ctx))


@dataclass
class MixedWorkload:
    """One chunked-prefill step at the attention boundary (decoders first)."""

    q: torch.Tensor  # bf16 [N, HQ, D] (post norm/rope)
    k: torch.Tensor  # bf16 [N, HKV, D]
    v: torch.Tensor  # bf16 [N, HKV, D], a strided view of a [N, 4096] qkv buffer
    cache: LayerKVCache
    inputs: dict  # int32 tensors: seq_ids, cu_seqlens, cached_lens, slot_ids, cu_cached, ...
    block_m: int
    decode_ctx: list
    chunks: list  # (chunk_len, cached_len) of the prefilling entries


def mixed_workload(decode_ctx: list, chunks: list, seed: int = 0, block_m: int = 128,
                   max_len: int = 4096, num_entries: int | None = None, pool: int | None = None,
                   n_pad: int | None = None, device="cpu", hq: int = HQ,
                   hkv: int = HKV) -> MixedWorkload:
    """Config-4-shaped step: decoders with `decode_ctx` tokens attended, then prefill chunks
    (chunk_len, cached_len). A prefilling entry's cached prefix is filled with calibration
    (its first chunk computed one), decoders' rows without. Entry b uses cache slot b; the
    last slot of the pool (default num_entries + 1 slots) is the scratch slot of the padding
    and unused entries. n_pad (default: the token count) pads the step to a token bucket. hq,
    hkv: query and KV heads (default 16 and 8)."""
    gen = torch.Generator().manual_seed(seed)
    nd = len(decode_ctx)
    B = nd + len(chunks)
    S = num_entries or B + 1
    pool = pool or S + 1
    assert pool > B
    scratch = pool - 1
    cache = empty_cache(pool, max_len, hkv=hkv)
    plan = []
    for i, c in enumerate(decode_ctx):
        fill_rows(cache, i, c - 1, gen)  # the new token is written by fused_rope_kv_decode
        plan.append((c - 1, i, [0]))
    for j, (L, cached) in enumerate(chunks):
        slot = nd + j
        fill_rows(cache, slot, cached, gen, calibrate=True)
        plan.append((cached, slot, [0] * L))
    N = n_pad or sum(len(t) for _, _, t in plan)
    step = fill_inputs(plan, nd, N, S, block_m, scratch)
    qkv = randn_bf16((N, (hq + 2 * hkv) * D), gen)
    q = qkv[:, : hq * D].reshape(N, hq, D).contiguous()
    k = qkv[:, hq * D:(hq + hkv) * D].reshape(N, hkv, D).contiguous()
    v = qkv.view(N, hq + 2 * hkv, D)[:, hq + hkv:]
    inputs = step.to_device("cpu")
    wl = MixedWorkload(q, k, v, cache, inputs, block_m, list(decode_ctx), list(chunks))
    return wl if device == "cpu" else mixed_to(wl, device)


def mixed_to(wl: MixedWorkload, device) -> MixedWorkload:
    c = wl.cache
    qkv_v = wl.v.to(device) if wl.v.is_contiguous() else None
    if qkv_v is None:  # keep v a strided view with the same token stride
        N, hq, hkv = wl.v.shape[0], wl.q.shape[1], wl.k.shape[1]
        base = torch.empty(N, (hq + 2 * hkv), D, dtype=wl.v.dtype, device=device)
        base[:, hq + hkv:] = wl.v.to(device)
        qkv_v = base[:, hq + hkv:]
    return MixedWorkload(
        wl.q.to(device), wl.k.to(device), qkv_v,
        LayerKVCache(*(t.to(device) for t in (c.k, c.v, c.k_scale, c.v_scale, c.k_calibration))),
        {n: t.to(device) for n, t in wl.inputs.items()}, wl.block_m, wl.decode_ctx, wl.chunks)


def config4(seed: int = 0, block_m: int = 128) -> MixedWorkload:
    """30 decoders (ctx ~ U[128, 2048]), chunk A (512 new, 0 cached),
    chunk B (512 new, 1536 cached)."""
    g = torch.Generator().manual_seed(seed + 7)
    dctx = torch.randint(128, 2049, (30,), generator=g).tolist()
    return mixed_workload(dctx, [(512, 0), (512, 1536)], seed=seed, block_m=block_m)


def prefill_flops(chunks: list, hq: int = HQ, d: int = D) -> int:
    """Causal-exact attention flops (QK^T + PV) of prefill chunks (chunk_len, cached_len)."""
    pairs = sum(L * c + L * (L + 1) // 2 for L, c in chunks)
    return 4 * hq * d * pairs
