"""Oracle for the per-layer residual/norm and activation kernels (test infrastructure only; see
oracle/__init__.py).

Restates qwen3-1.7b/kernels.py:
  add_rms_norm  :1216-1283  new_residual = bf16(residual + delta) (fp32 add);
                            normed = bf16((r * rsqrt(sum(r^2) / D + eps)) * w), r = new_residual
  silu_mul      :1178-1213  [N, 2D] -> [N, D]: bf16((gate * sigmoid(gate)) * up), fp32

The reference leaves the order of sum(r^2) to Triton's tl.sum; this build fixes it (the HIP
kernel's order): thread t of a 256-thread workgroup owns elements 8t + 2048j + i (j = 0, 1, ...;
i = 0..7) and adds their squares in that order, the 64 threads of each wave are combined by the
xor butterfly (lane distance 32, 16, ..., 1), and the four wave sums are added in wave order.
rsqrt is 1 / sqrt, both IEEE. The reference's tl.rsqrt and tl.sigmoid lower to the NVIDIA
target's approximations, which cannot be observed here: parity with the reference is at
float64 level (one bf16 rounding), and the HIP kernel matches this restatement bit for bit for
add_rms_norm and to one bf16 unit for silu_mul (its exp is the device's, not numpy's).
"""

import numpy as np

from .numerics import F32, bf16_round, butterfly_sum64

NORM_THREADS = 256
NORM_VEC = 8


def sum_squares(r):
    """sum of r^2 over the last axis (length D, a multiple of 8) in the kernel's order."""
    r = np.asarray(r, np.float32)
    *lead, D = r.shape
    assert D % NORM_VEC == 0
    step = NORM_THREADS * NORM_VEC
    per_thread = np.zeros((*lead, NORM_THREADS), np.float32)
    for j in range(0, D, step):
        for i in range(NORM_VEC):
            idx = j + NORM_VEC * np.arange(NORM_THREADS) + i
            ok = idx < D
            v = np.where(ok, r[..., np.minimum(idx, D - 1)], F32(0))
            per_thread = np.where(ok, (per_thread + (v * v).astype(np.float32)).astype(np.float32),
                                  per_thread)
    waves = butterfly_sum64(per_thread.reshape(*lead, NORM_THREADS // 64, 64))  # [..., 4]
    total = waves[..., 0]
    for w in range(1, NORM_THREADS // 64):
        total = (total + waves[..., w]).astype(np.float32)
    return total


def add_rms_norm(residual, delta, weight, eps):
    """(new_residual, normed), both fp32 values of bf16 results; inputs fp32 values of bf16."""
    res = bf16_round((np.asarray(residual, np.float32) + np.asarray(delta, np.float32))
                     .astype(np.float32))
    D = res.shape[-1]
    var = (sum_squares(res) / F32(D) + F32(eps)).astype(np.float32)
    inv = (F32(1.0) / np.sqrt(var)).astype(np.float32)[..., None]
    w = np.asarray(weight, np.float32)
    normed = bf16_round(((res * inv).astype(np.float32) * w).astype(np.float32))
    return res, normed


def silu_mul(gate_up):
    """[N, 2D] -> [N, D] fp32 values of the bf16 result."""
    x = np.asarray(gate_up, np.float32)
    D = x.shape[-1] // 2
    gate, up = x[..., :D], x[..., D:]
    sig = (F32(1.0) / (F32(1.0) + np.exp(-gate).astype(np.float32))).astype(np.float32)
    return bf16_round(((gate * sig).astype(np.float32) * up).astype(np.float32))
