"""skinny_matmul / linear / tune_linear (qwen3-1.7b/kernels.py:1373-1485) on the GPU: y = x W^T
for decode row counts against a float32 matmul (each output within one bf16 rounding of the
fp32 value, up to fp32 summation-order noise), for every n_tiles launch shape, Qwen3-1.7B's
projection shapes and ragged row counts; linear follows the table tune_linear fills."""

import pytest
import torch

from helpers import say

SHAPES = [(4096, 2048), (2048, 2048), (12288, 2048), (2048, 6144), (512, 256)]


def _check(y, x, w, what):
    ref = x.float() @ w.float().T
    # one bf16 rounding of the exact value: |y - ref| <= 2^-8 |ref| (+ fp32 summation noise)
    err = (y.float() - ref).abs()
    bound = ref.abs() * 2 ** -8 + 1e-3 * ref.abs().max()
    assert torch.all(err <= bound), f"{what}: max err {err.max().item():.3e}"


@pytest.mark.gpu
@pytest.mark.parametrize("N,K", SHAPES)
@pytest.mark.parametrize("M", [1, 8, 17, 32, 64])
def test_skinny_matmul(ie, dev, N, K, M):
    g = torch.Generator().manual_seed(N + K + M)
    w = (0.02 * torch.randn(N, K, generator=g)).bfloat16().to(dev)
    x = torch.randn(M, K, generator=g).bfloat16().to(dev)
    for nt in (0, 1, 2, 4):
        if N % (16 * max(1, nt)):
            continue
        y = ie.skinny_matmul(x, w, nt)
        torch.cuda.synchronize()
        assert y.shape == (M, N) and y.dtype == torch.bfloat16
        _check(y, x, w, f"N={N} K={K} M={M} n_tiles={nt}")
    say(f"skinny_matmul N={N} K={K} M={M}: ok")


@pytest.mark.gpu
def test_strided_x_rows(ie, dev):
    g = torch.Generator().manual_seed(1)
    w = (0.02 * torch.randn(2048, 2048, generator=g)).bfloat16().to(dev)
    wide = torch.randn(16, 4096, generator=g).bfloat16().to(dev)
    x = wide[:, 1024:3072]  # row stride 4096
    _check(ie.skinny_matmul(x, w), x, w, "strided x")


@pytest.mark.gpu
def test_linear_follows_tuning_table(ie, dev):
    g = torch.Generator().manual_seed(2)
    w = (0.02 * torch.randn(4096, 2048, generator=g)).bfloat16().to(dev)
    K = ie.kernels
    tables = (K.use_skinny, K.use_skinny_glu, K.use_skinny_swz, K.use_skinny_glu_swz)
    for t in tables:
        t.clear()
    K.tune_linear([w], [8, 32, 100])
    assert (4096, 2048, 100) not in K.use_skinny  # > 64 rows: always the library
    assert K.use_skinny[(4096, 2048, 8)] in (None, 0, 1, 2, 4)
    if K.use_skinny[(4096, 2048, 8)] is not None:
        assert K.use_skinny_glu[(4096, 2048, 8)] in (1, 2)
        assert K.swizzled_tiles(4096, 2048, 8) in (None, 1, 2, 4)
        assert K.swizzled_tiles(4096, 2048, 8, True) in (None, 1, 2)
    say(f"tuned: {K.use_skinny} swizzled: {K.use_skinny_swz} {K.use_skinny_glu_swz}")
    for M in (8, 32, 100):
        x = torch.randn(M, 2048, generator=g).bfloat16().to(dev)
        _check(K.linear(x, w), x, w, f"linear M={M}")
        nt = K.swizzled_tiles(4096, 2048, M)
        if nt is not None:  # the reordered weight at the width tuned for it
            sw = K.swizzle_weight(w, nt)
            _check(K.skinny_matmul(x, sw, nt, swizzled=True), x, w, f"swizzled M={M} nt={nt}")
    for t in tables:
        t.clear()


def _check_glu(y, x, w, what):
    D = w.shape[0] // 2
    gu = x.float() @ w.float().T
    g, u = gu[:, :D].bfloat16().float(), gu[:, D:].bfloat16().float()
    ref = (g * torch.sigmoid(g)) * u
    # one bf16 rounding of the product, plus the bf16 roundings of g and u when the fp32 sums
    # land on the other side of a rounding boundary
    err = (y.float() - ref).abs()
    bound = ref.abs() * 2 ** -7 + 2e-3 * ref.abs().max()
    assert torch.all(err <= bound), f"{what}: max err {err.max().item():.3e}"


@pytest.mark.gpu
@pytest.mark.parametrize("N,K", [(12288, 2048), (1024, 512)])
@pytest.mark.parametrize("M", [1, 17, 32, 64])
def test_skinny_matmul_silu_mul(ie, dev, N, K, M):
    g = torch.Generator().manual_seed(N + K + M + 1)
    w = (0.02 * torch.randn(N, K, generator=g)).bfloat16().to(dev)
    x = torch.randn(M, K, generator=g).bfloat16().to(dev)
    for nt in (1, 2):
        y = ie.skinny_matmul_silu_mul(x, w, nt)
        torch.cuda.synchronize()
        assert y.shape == (M, N // 2) and y.dtype == torch.bfloat16
        _check_glu(y, x, w, f"fused N={N} K={K} M={M} n_tiles={nt}")
        # the two-launch path it replaces
        two = ie.silu_mul(ie.skinny_matmul(x, w, nt))
        torch.cuda.synchronize()
        _check_glu(two, x, w, f"two-step N={N} K={K} M={M}")
    say(f"skinny_matmul_silu_mul N={N} K={K} M={M}: ok")


@pytest.mark.gpu
def test_linear_silu_mul_follows_tuning_table(ie, dev):
    g = torch.Generator().manual_seed(4)
    w = (0.02 * torch.randn(1024, 512, generator=g)).bfloat16().to(dev)
    x = torch.randn(8, 512, generator=g).bfloat16().to(dev)
    K = ie.kernels
    for choice in (None, 1, 4):  # library, then the fused skinny launch
        K.use_skinny[(1024, 512, 8)] = choice
        _check_glu(K.linear_silu_mul(x, w), x, w, f"linear_silu_mul table={choice}")
    for nt in (1, 2):  # the fused launch's own tuned width takes precedence
        K.use_skinny_glu[(1024, 512, 8)] = nt
        _check_glu(K.linear_silu_mul(x, w), x, w, f"linear_silu_mul glu table={nt}")
    K.use_skinny.pop((1024, 512, 8))
    K.use_skinny_glu.pop((1024, 512, 8))
