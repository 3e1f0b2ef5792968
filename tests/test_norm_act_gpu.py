"""add_rms_norm / silu_mul (qwen3-1.7b/kernels.py:1178-1283) on the GPU against the oracle: the new
residual and the normed rows bit-exact (Qwen3's 2048, the 6144-wide intermediate, a single
8-wide row, strided rows), silu_mul within one bf16 unit (the device's exp is not numpy's) and
almost always exact."""

import numpy as np
import pytest
import torch

from helpers import bf16_np, say
from oracle import norm_act as ona
from oracle.numerics import bf16_bits


def _bf16(shape, seed, dev, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (scale * torch.randn(*shape, generator=g)).bfloat16().to(dev)


@pytest.mark.gpu
@pytest.mark.parametrize("N,D", [(32, 2048), (5, 6144), (3, 8), (1, 8192)])
def test_add_rms_norm_bitexact(ie, dev, N, D):
    say(f"add_rms_norm N={N} D={D}")
    wide = _bf16((N, D + 64), N + D, dev, 3.0)
    res = wide[:, 32:32 + D]  # a strided view
    delta = _bf16((N, D), 2, dev)
    w = (1 + 0.1 * _bf16((D,), 3, dev).float()).bfloat16()
    nres, normed = ie.add_rms_norm(res, delta, w, 1e-6)
    torch.cuda.synchronize()
    rr, rn = ona.add_rms_norm(bf16_np(res), bf16_np(delta), bf16_np(w), 1e-6)
    assert np.array_equal(bf16_bits(bf16_np(nres)), bf16_bits(rr))
    bad = np.argwhere(bf16_bits(bf16_np(normed)) != bf16_bits(rn))
    assert bad.size == 0, f"{len(bad)} mismatches, first {bad[:4].tolist()}"


@pytest.mark.gpu
@pytest.mark.parametrize("N,D", [(32, 6144), (3, 8), (2, 2056)])
def test_silu_mul_close(ie, dev, N, D):
    say(f"silu_mul N={N} D={D}")
    gu = _bf16((N, 2 * D), 5 + D, dev, 4.0)
    out = ie.silu_mul(gu)
    torch.cuda.synchronize()
    ref = ona.silu_mul(bf16_np(gu))
    got = bf16_np(out)
    assert out.shape == (N, D)
    ulp = np.abs(bf16_bits(got).astype(np.int64) - bf16_bits(ref).astype(np.int64))
    same_sign = np.sign(got) == np.sign(ref)
    assert np.all((ulp <= 1) & (same_sign | (got == 0) | (ref == 0)))
    assert (ulp == 0).mean() > 0.999
    say(f"silu_mul: {(ulp == 0).mean():.5f} exact")


@pytest.mark.gpu
def test_empty_rows(ie, dev):
    r = _bf16((0, 2048), 1, dev)
    w = _bf16((2048,), 2, dev)
    a, b = ie.add_rms_norm(r, r, w, 1e-6)
    c = ie.silu_mul(_bf16((0, 4096), 3, dev))
    torch.cuda.synchronize()
    assert a.shape == (0, 2048) and b.shape == (0, 2048) and c.shape == (0, 2048)


@pytest.mark.gpu
def test_rope_tables_match_pytorch(ie, dev):
    """attention_layer.rope_tables (one HIP launch) against the reference's PyTorch arithmetic
    (architecture.py:382-390: int32 positions times the fp32 inverse frequencies, cos and sin,
    cast to bf16) on the device, bit for bit: positions 0 .. 70,000 and a decode step's
    cached lengths, head_dim 128 (rope base 1e6) and 64 (base 1e4)."""
    al = ie.attention_layer
    g = torch.Generator().manual_seed(9)
    for D, base in ((128, 1e6), (64, 1e4)):
        inv = al.rope_inv_freq(D, base, dev)
        for pos in (torch.arange(70000, dtype=torch.int32),
                    torch.randint(0, 40000, (33,), generator=g, dtype=torch.int32)):
            p = pos.to(dev)
            c, s = al.rope_tables(p, inv)
            ang = p[:, None, None] * inv[None, None, :]
            rc, rs = ang.cos().to(torch.bfloat16), ang.sin().to(torch.bfloat16)
            torch.cuda.synchronize()
            assert c.shape == rc.shape and s.shape == rs.shape
            dc = (c.view(torch.int16) != rc.view(torch.int16)).sum().item()
            dsn = (s.view(torch.int16) != rs.view(torch.int16)).sum().item()
            assert dc == 0 and dsn == 0, f"D={D}: {dc} cos, {dsn} sin entries differ"
