"""Pins the add_rms_norm / silu_mul oracle (oracle/norm_act.py, qwen3-1.7b/kernels.py:1178-1283) on
the CPU: float64 RMSNorm and SiLU within one bf16 rounding, the bf16 residual add against
torch, and known answers."""

import numpy as np
import torch

from oracle import norm_act as ona
from oracle.numerics import bf16_round

F32 = np.float32


def _bf16(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (scale * torch.randn(*shape, generator=g)).bfloat16()


def test_sum_squares_is_a_sum():
    x = _bf16((5, 6144), 0).float().numpy()
    ref = (x.astype(np.float64) ** 2).sum(axis=-1)
    assert np.allclose(ona.sum_squares(x), ref, rtol=1e-5)
    assert ona.sum_squares(np.ones((1, 2048), np.float32))[0] == F32(2048.0)
    assert ona.sum_squares(np.full((1, 8), 3.0, np.float32))[0] == F32(72.0)


def test_add_rms_norm_matches_float64():
    N, D = 9, 2048
    res, delta = _bf16((N, D), 1, 3.0), _bf16((N, D), 2)
    w = (1 + 0.1 * torch.randn(D, generator=torch.Generator().manual_seed(3))).bfloat16()
    nres, normed = ona.add_rms_norm(res.float().numpy(), delta.float().numpy(), w.float().numpy(),
                                    1e-6)
    # the new residual is torch's bf16 add (fp32 add, one rounding)
    assert np.array_equal(nres, (res + delta).float().numpy())
    r64 = nres.astype(np.float64)
    ref = r64 / np.sqrt((r64 ** 2).mean(axis=-1, keepdims=True) + 1e-6) * w.double().numpy()
    assert np.all(np.abs(normed - ref) <= 2 ** -8 * np.abs(ref) + 1e-6)
    assert np.array_equal(normed, bf16_round(normed))


def test_add_rms_norm_known_answers():
    D = 16
    res = np.zeros((3, D), np.float32)
    res[0] = 2.0  # constant row: rms 2 -> normed = w (eps 0)
    res[1, :8], res[1, 8:] = 1.0, -1.0  # rms 1
    w = np.full(D, 0.5, np.float32)
    nres, normed = ona.add_rms_norm(res[:2], np.zeros_like(res[:2]), w, 0.0)
    assert np.array_equal(nres, res[:2])
    assert np.all(normed[0] == 0.5)
    assert np.all(normed[1, :8] == 0.5) and np.all(normed[1, 8:] == -0.5)
    # a zero row with eps: 0 * (1 / sqrt(eps)) * w = 0
    _, n2 = ona.add_rms_norm(res, np.zeros_like(res), w, 1e-6)
    assert np.all(n2[2] == 0.0)


def test_silu_mul_matches_float64_and_known_answers():
    N, D = 7, 6144
    gu = _bf16((N, 2 * D), 4, 4.0).float().numpy()
    out = ona.silu_mul(gu)
    g, u = gu[:, :D].astype(np.float64), gu[:, D:].astype(np.float64)
    ref = g / (1 + np.exp(-g)) * u
    assert np.all(np.abs(out - ref) <= 2 ** -8 * np.abs(ref) + 1e-6)
    x = np.array([[0.0, 50.0, -50.0, 2.0, 1.0, 1.0, 3.0, 1.0]], np.float32)  # gates | ups
    y = ona.silu_mul(x)
    assert y[0, 0] == 0.0 and y[0, 1] == 50.0  # silu(0) = 0, silu(50) = 50
    assert abs(y[0, 2]) < 1e-19  # silu(-50) ~ -1e-20
    assert y[0, 3] == bf16_round(np.float32(2.0 / (1 + np.exp(-2.0))))
