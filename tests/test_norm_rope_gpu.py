"""fused_norm_rope_prefill (qwen3-1.7b/kernels.py:547-714) on the GPU against the oracle: bit-exact
bf16 outputs for strided q/k views of a fused qkv row, ragged and config-4-sized token counts, an
empty batch, and agreement with the decode write's own norm + rope of the same rows."""

import numpy as np
import pytest
import torch

from helpers import bf16_np, say
from oracle import kv_cache as okv
from oracle.numerics import bf16_bits


def _inputs(N, seed, dev, hq=16, hkv=8, scale=2.0):
    g = torch.Generator().manual_seed(seed)
    qkv = (scale * torch.randn(N, (hq + 2 * hkv) * 128, generator=g)).bfloat16()
    qw = (1 + 0.1 * torch.randn(128, generator=g)).bfloat16()
    kw = (1 + 0.1 * torch.randn(128, generator=g)).bfloat16()
    pos = torch.randint(0, 40000, (N,), generator=g).float()
    inv = 1e6 ** (-torch.arange(0, 128, 2, dtype=torch.float32) / 128)
    ang = pos[:, None, None] * inv[None, None, :]
    cos, sin = ang.cos().bfloat16(), ang.sin().bfloat16()
    qkv, qw, kw, cos, sin = (t.to(dev) for t in (qkv, qw, kw, cos, sin))
    q = qkv[:, :hq * 128].view(N, hq, 128)
    k = qkv[:, hq * 128:(hq + hkv) * 128].view(N, hkv, 128)
    return q, k, qw, kw, cos, sin


def _check(ie, q, k, qw, kw, cos, sin, what):
    q_out, k_out = ie.fused_norm_rope_prefill(q, k, qw, kw, cos, sin, 1e-6)
    torch.cuda.synchronize()
    assert q_out.shape == q.shape and k_out.shape == k.shape
    assert q_out.is_contiguous() and k_out.is_contiguous()
    rq, rk = okv.fused_norm_rope_prefill(*(bf16_np(t) for t in (q, k, qw, kw, cos, sin)), 1e-6)
    for name, got, ref in (("q", q_out, rq), ("k", k_out, rk)):
        bad = np.argwhere(bf16_bits(bf16_np(got)) != bf16_bits(ref))
        assert bad.size == 0, f"{what} {name}: {len(bad)} mismatches, first {bad[:4].tolist()}"
    say(f"{what}: bit-exact")


@pytest.mark.gpu
@pytest.mark.parametrize("N", [1, 37, 1054])
def test_norm_rope_prefill_bitexact(ie, dev, N):
    say(f"norm_rope_prefill N={N}")
    _check(ie, *_inputs(N, 100 + N, dev), f"N={N}")


@pytest.mark.gpu
def test_norm_rope_prefill_other_head_counts(ie, dev):
    # a tensor-parallel shard's heads (Hq 4, Hkv 2) and more rows than one workgroup covers
    for hq, hkv in ((4, 2), (32, 8)):
        say(f"norm_rope_prefill Hq={hq} Hkv={hkv}")
        _check(ie, *_inputs(29, 7, dev, hq=hq, hkv=hkv), f"Hq={hq} Hkv={hkv}")


@pytest.mark.gpu
def test_norm_rope_prefill_extreme_rows(ie, dev):
    # a zero row (rstd = 1/sqrt(eps)), huge and tiny magnitudes
    q, k, qw, kw, cos, sin = _inputs(5, 9, dev)
    q, k = q.clone(), k.clone()
    q[0, 3].zero_()
    q[1] *= 3000
    k[2] *= 1e-3
    say("norm_rope_prefill extreme rows")
    _check(ie, q, k, qw, kw, cos, sin, "extreme rows")


@pytest.mark.gpu
def test_norm_rope_prefill_empty(ie, dev):
    q, k, qw, kw, cos, sin = _inputs(1, 3, dev)
    q_out, k_out = ie.fused_norm_rope_prefill(q[:0], k[:0], qw, kw, cos[:0], sin[:0], 1e-6)
    torch.cuda.synchronize()
    assert q_out.shape == (0, 16, 128) and k_out.shape == (0, 8, 128)


@pytest.mark.gpu
def test_norm_rope_prefill_matches_decode_rotation(ie, dev):
    # with calibration ones, the decode write's q output is the same norm + rope
    B = 8
    q, k, qw, kw, cos, sin = _inputs(B, 11, dev)
    cache = ie.make_layer_cache(B, 8, 4, 128, device=dev)
    i32 = lambda x: torch.tensor(x, dtype=torch.int32, device=dev)
    qd = ie.fused_rope_kv_decode(q, k, k, qw, kw, cos, sin, i32(list(range(B))), cache,
                                 i32([0] * B), i32([B]), 1e-6)
    qp, _ = ie.fused_norm_rope_prefill(q, k, qw, kw, cos, sin, 1e-6)
    torch.cuda.synchronize()
    say("norm_rope_prefill vs decode rotation")
    assert torch.equal(qd, qp)
