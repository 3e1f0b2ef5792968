"""Rounding helpers shared by the oracle (test infrastructure only; see oracle/__init__.py)."""

import numpy as np

F32 = np.float32


def bf16_round(x) -> np.ndarray:
    """fp32 -> bf16 -> fp32 with round-to-nearest-even, NaN preserved.

    This is the rounding of Triton's `.to(tl.bfloat16)` / bf16 `tl.store` used throughout
    qwen3-1.7b/kernels.py (e.g. :186, :924, :930, :1068).
    """
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    bias = ((u >> 16) & 1) + 0x7FFF
    r = ((u + bias) & 0xFFFF0000).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, r).astype(np.float32)


def bf16_bits(x) -> np.ndarray:
    """Bit pattern (uint16) of the bf16 value nearest to fp32 `x`."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bits_to_f32(bits) -> np.ndarray:
    """bf16 bit patterns (uint16) -> exact fp32 values."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def butterfly_sum64(x) -> np.ndarray:
    """Sum over the last axis (length 64) in the order of a wave64 xor-butterfly.

    Lane i adds lane i^32, then i^16, 8, 4, 2, 1; every lane ends with the same fp32 value.
    This fixes the summation order the HIP kernel uses for the RMSNorm sum of squares, which
    the reference leaves to Triton's `tl.sum` (qwen3-1.7b/kernels.py:417,426).
    """
    x = np.asarray(x, dtype=np.float32)
    assert x.shape[-1] == 64
    idx = np.arange(64)
    for off in (32, 16, 8, 4, 2, 1):
        x = (x + x[..., idx ^ off]).astype(np.float32)
    return x[..., 0]
