"""Oracle for token sampling (test infrastructure only; see oracle/__init__.py).

Restates qwen3-1.7b/kernels.py:1286-1370 (`sampling_kernel`, `combine_partial_samples_kernel`,
`sample`): Gumbel-max sampling, token = argmax_v (logits[b, v] + tau * -log(-log(u[b, v]))), the
first index winning ties (Triton's `tl.max(..., return_indices=True)` within a block, then the
first block), then seed += 1. With tau = 0 the noise term is 0 * finite and the result is the
greedy argmax.

The uniforms are Triton's `tl.rand(seed, offset)` with offset = b * V + v (int32), which is
Philox4x32-10 (Salmon et al., "Parallel random numbers: as easy as 1, 2, 3", SC11; the Random123
reference implementation) on counter (offset, 0, 0, 0) and key (seed low 32 bits, seed high 32
bits), taking the first output word as int32 x and mapping it to
float32(x < 0 ? -x - 1 : x) * float32(4.6566127342e-10) (triton/language/random.py of the
triton package the reference pins, uv.lock:931-932; the algorithm is restated here, not
imported). The uniform is clamped to [1e-10, 1 - 1e-7] (kernels.py:1308).
"""

import numpy as np

PHILOX_M0, PHILOX_M1 = 0xD2511F53, 0xCD9E8D57  # round multipliers
PHILOX_W0, PHILOX_W1 = 0x9E3779B9, 0xBB67AE85  # key increments (Weyl sequence)
U32 = np.uint64(0xFFFFFFFF)
UNIFORM_SCALE = np.float32(4.6566127342e-10)
U_LO, U_HI = np.float32(1e-10), np.float32(1.0 - 1e-7)


def philox4x32(c0, c1, c2, c3, k0, k1, rounds=10):
    """Philox4x32 on uint32 arrays (carried in uint64): returns the four output words."""
    c = [np.asarray(x, np.uint64) & U32 for x in (c0, c1, c2, c3)]
    k0, k1 = np.uint64(k0) & U32, np.uint64(k1) & U32
    for _ in range(rounds):
        p0 = np.uint64(PHILOX_M0) * c[0]
        p1 = np.uint64(PHILOX_M1) * c[2]
        c = [(p1 >> np.uint64(32)) ^ c[1] ^ k0, p1 & U32, (p0 >> np.uint64(32)) ^ c[3] ^ k1, p0 & U32]
        k0 = (k0 + np.uint64(PHILOX_W0)) & U32
        k1 = (k1 + np.uint64(PHILOX_W1)) & U32
    return c


def uniform_from_u32(x):
    """triton uint_to_uniform_float for 32-bit words: float in [0, 1)."""
    i = np.asarray(x, np.uint64).astype(np.uint32).view(np.int32).astype(np.int64)
    i = np.where(i < 0, -i - 1, i)
    return (i.astype(np.float32) * UNIFORM_SCALE).astype(np.float32)


def rand(seed, offsets):
    """tl.rand(seed, offsets) for int32 offsets and an int64 seed."""
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    off = np.asarray(offsets, np.int64).astype(np.uint32).astype(np.uint64)
    z = np.zeros_like(off)
    c0, _, _, _ = philox4x32(off, z, z, z, seed & 0xFFFFFFFF, seed >> 32)
    return uniform_from_u32(c0)


def gumbel_logits(logits, tau, seed):
    """logits + tau * -log(-log(clamp(u))) in float32, as kernels.py:1305-1310."""
    x = np.asarray(logits, np.float32)
    B, V = x.shape
    off = (np.arange(B, dtype=np.int64)[:, None] * V + np.arange(V, dtype=np.int64)[None, :])
    off = off.astype(np.uint64).astype(np.uint32).view(np.int32)  # int32 wrap-around
    u = np.clip(rand(seed, off), U_LO, U_HI).astype(np.float32)
    g = (-np.log((-np.log(u)).astype(np.float32))).astype(np.float32)
    return (x + (np.float32(tau) * g).astype(np.float32)).astype(np.float32)


def sample(logits, tau, seed):
    """Returns (tokens int64 [B, 1], next seed). The first maximal index wins."""
    x = gumbel_logits(logits, tau, seed)
    return np.argmax(x, axis=1).astype(np.int64)[:, None], int(seed) + 1
