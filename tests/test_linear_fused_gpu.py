"""The skinny GEMM with a decoder layer's residual add and RMSNorm fused in (ie_skinny_gemm_fused,
`linear_residual_`, `linear_norm`), which the decode step uses in place of the reference's
add_rms_norm launches between its projections (qwen3-1.7b/kernels.py:1216-1283 at
architecture.py:280-300):

* the residual form is add_rms_norm's new residual bit for bit, given the plain GEMM's output:
  bf16(residual + bf16(x W^T)) with the plain launch of the same tile width;
* the norm form against the oracle's add_rms_norm followed by a float32 matmul, under a bound
  that holds for any summation order: the folded weight bf16(g W) and the oracle's normalized
  row bf16(h rstd g) each round one factor of every product once (at most 2^-9 relative each),
  and the output is rounded once more;
* rstd exactly as add_rms_norm computes it (IEEE 1 / sqrt(sum / K + eps)): rows with two nonzero
  entries at opposite ends of K (summed by different waves) against integer weights, where
  every product and sum is exact and the expected output is known bit for bit;
* the gate/up form against the norm form's output passed through silu_mul.
"""

import numpy as np
import pytest
import torch

from helpers import bf16_np, say
from oracle import norm_act as ona
from oracle.numerics import bf16_bits

pytestmark = pytest.mark.gpu
SHAPES = [(4096, 2048), (2048, 2048), (2048, 6144), (512, 256)]
EPS = 1e-6


def _tiles(N):
    return [nt for nt in (0, 1, 2, 4) if N % (16 * max(1, nt)) == 0]


@pytest.mark.parametrize("N,K", SHAPES)
@pytest.mark.parametrize("M", [1, 17, 32, 64])
def test_residual_form_is_add_rms_norm_residual(ie, dev, N, K, M):
    g = torch.Generator().manual_seed(N + K + M + 100)
    w = (0.02 * torch.randn(N, K, generator=g)).bfloat16().to(dev)
    x = torch.randn(M, K, generator=g).bfloat16().to(dev)
    res0 = (3 * torch.randn(M, N, generator=g)).bfloat16().to(dev)
    K_ = ie.kernels
    for nt in _tiles(N):
        y = ie.skinny_matmul(x, w, nt)
        res = res0.clone()
        out = K_.ops().skinny_matmul_residual_(x, w, nt, res)
        torch.cuda.synchronize()
        assert out.data_ptr() == res.data_ptr()
        want, _ = ona.add_rms_norm(bf16_np(res0), bf16_np(y), np.ones(N, np.float32), EPS)
        bad = np.argwhere(bf16_bits(bf16_np(res)) != bf16_bits(want))
        assert bad.size == 0, f"N={N} K={K} M={M} nt={nt}: {len(bad)} mismatches {bad[:4]}"
    say(f"residual form N={N} K={K} M={M}: bit-exact")


def _norm_inputs(M, K, N, seed, dev):
    g = torch.Generator().manual_seed(seed)
    h = (2 * torch.randn(M, K, generator=g)).bfloat16()
    if M > 2:  # a large and a tiny row (rstd far from 1 both ways)
        h[1] *= 300
        h[2] *= 1e-3
    gam = (1 + 0.3 * torch.randn(K, generator=g)).bfloat16()
    w = (0.02 * torch.randn(N, K, generator=g)).bfloat16()
    return h.to(dev), gam.to(dev), w.to(dev)


def _check_norm(y, h, gam, w, what):
    """|y - ref| <= 2^-8 * sum_k |h_k rstd g_k W_nk| + 2^-8 |ref|, ref = bf16 normalized rows of
    the oracle's add_rms_norm times W in float32 (2^-8 covers the two 2^-9 roundings)."""
    M, K = h.shape
    _, normed = ona.add_rms_norm(bf16_np(h), np.zeros(h.shape, np.float32), bf16_np(gam), EPS)
    ref = normed.astype(np.float64) @ bf16_np(w).astype(np.float64).T
    _, nrm1 = ona.add_rms_norm(bf16_np(h), np.zeros(h.shape, np.float32), np.ones(K, np.float32),
                               EPS)  # h * rstd without the weight, bf16-rounded
    absterm = np.abs(nrm1).astype(np.float64) @ np.abs(
        bf16_np(gam).astype(np.float64)[None, :] * bf16_np(w).astype(np.float64)).T
    err = np.abs(bf16_np(y).astype(np.float64) - ref)
    bound = 2.0 ** -8 * (absterm * 1.01 + np.abs(ref)) + 1e-30
    assert np.all(err <= bound), f"{what}: max err/bound {np.max(err / bound):.3f}"


@pytest.mark.parametrize("N,K", SHAPES)
@pytest.mark.parametrize("M", [1, 17, 32, 64])
def test_norm_form_against_oracle(ie, dev, N, K, M):
    h, gam, w = _norm_inputs(M, K, N, N + K + M + 200, dev)
    wf = ie.fold_rms_norm_weight(w, gam)
    for nt in _tiles(N):
        y = ie.kernels.ops().skinny_matmul_norm(h, wf, nt, False, EPS)
        torch.cuda.synchronize()
        assert y.shape == (M, N)
        _check_norm(y, h, gam, w, f"norm form N={N} K={K} M={M} nt={nt}")
    say(f"norm form N={N} K={K} M={M}: ok")


@pytest.mark.parametrize("K", [256, 2048, 6144])
def test_norm_form_rstd_exact(ie, dev, K):
    """Row m holds a_m at k = 3 (the first wave's slice) and b_m at k = K - 5 (the last
    wave's), W' small integers: a W'_3 + b W'_(K-5) and a^2 + b^2 are exact in float32, so the
    output is bf16(rstd * that) with rstd = 1 / sqrt((a^2 + b^2) / K + eps), bit for bit."""
    M, N = 20, 64
    g = torch.Generator().manual_seed(K)
    a = torch.tensor([1.5, -2.0, 0.25, 3.0, 0.0] * 4)
    b = torch.tensor([-2.0, 0.5, 0.0, 96.0, 0.125] * 4)
    h = torch.zeros(M, K)
    h[:, 3], h[:, K - 5] = a, b
    wf = torch.randint(-8, 9, (N, K), generator=g).float()
    y = ie.kernels.ops().skinny_matmul_norm(h.bfloat16().to(dev), wf.bfloat16().to(dev), 1,
                                            False, EPS)
    torch.cuda.synchronize()
    f32 = np.float32
    an, bn, wn = a.numpy().astype(f32), b.numpy().astype(f32), wf.numpy().astype(f32)
    ss = an * an + bn * bn
    rstd = (f32(1) / np.sqrt((ss / f32(K) + f32(EPS)).astype(f32))).astype(f32)
    acc = an[:, None] * wn[None, :, 3] + bn[:, None] * wn[None, :, K - 5]
    want = (acc * rstd[:, None]).astype(f32)
    from oracle.numerics import bf16_round
    assert np.array_equal(bf16_bits(bf16_np(y)), bf16_bits(bf16_round(want))), f"K={K}"


@pytest.mark.parametrize("N,K", [(12288, 2048), (1024, 512)])
@pytest.mark.parametrize("M", [1, 17, 32, 64])
def test_norm_gate_up_form(ie, dev, N, K, M):
    h, gam, w = _norm_inputs(M, K, N, N + K + M + 300, dev)
    wf = ie.fold_rms_norm_weight(w, gam)
    for nt in (1, 2):
        y = ie.kernels.ops().skinny_matmul_norm(h, wf, nt, True, EPS)
        two = ie.silu_mul(ie.kernels.ops().skinny_matmul_norm(h, wf, nt, False, EPS))
        torch.cuda.synchronize()
        assert y.shape == (M, N // 2)
        ref = two.float()
        err = (y.float() - ref).abs()
        # the gate and up sums may round to neighbouring bf16 values (another summation order)
        bound = ref.abs() * 2 ** -7 + 2e-3 * ref.abs().max()
        assert torch.all(err <= bound), f"N={N} K={K} M={M} nt={nt}: {err.max().item():.3e}"
    say(f"norm gate/up form N={N} K={K} M={M}: ok")


def test_linear_wrappers_follow_tuning_table(ie, dev):
    """linear_norm / linear_residual_ take the tile width tune_linear chose (1 where none)."""
    K_ = ie.kernels
    h, gam, w = _norm_inputs(8, 512, 1024, 7, dev)
    wf = ie.fold_rms_norm_weight(w, gam)
    for choice in (None, 0, 2, 4):
        K_.use_skinny[(1024, 512, 8)] = choice
        _check_norm(K_.linear_norm(h, wf, EPS), h, gam, w, f"linear_norm table={choice}")
        res0 = torch.randn(8, 1024, device=dev).bfloat16()
        res = res0.clone()
        K_.linear_residual_(h, w, res)
        want = (res0.float() + K_.skinny_matmul(h, w, 1 if choice is None else choice).float())
        torch.cuda.synchronize()
        assert torch.equal(res, want.bfloat16()), f"linear_residual_ table={choice}"
    K_.use_skinny.pop((1024, 512, 8))



@pytest.mark.parametrize("nt,gate_up", [(1, False), (2, False), (4, False), (1, True),
                                        (2, True), (3, True), (4, True)])
def test_swizzle_layout(ie, dev, nt, gate_up):
    """swizzle_weight against the layout it documents, restated on the CPU: for tile width G,
    the 1 KB block of 16-row group R and 32-column step S, at block index
    ((R / G) K / 32 + S) G + R % G, holds at 16 bytes per lane 16 g + r row 16 R + r, columns
    32 S + 8 g .. +8 (a strided source too); gate_up: of the weight whose 16-row group R is
    gate rows 8 R .. 8 R + 7 then up rows N / 2 + 8 R .. (the [gate; up] rows paired)."""
    N, K = 192, 256
    g = torch.Generator().manual_seed(5)
    wide = torch.randn(N, K + 64, generator=g).bfloat16()
    w = wide[:, 32:32 + K]
    out = ie.swizzle_weight(w.to(dev), nt, gate_up=gate_up).cpu()
    if gate_up:  # the paired row order, then the same layout
        w = torch.stack([w[:N // 2].reshape(N // 16, 8, K), w[N // 2:].reshape(N // 16, 8, K)],
                        dim=1).reshape(N, K)
    want = (w.reshape(N // (16 * nt), nt, 16, K // 32, 4, 8)  # band, R % G, r, S, g, 8
            .permute(0, 3, 1, 4, 2, 5)                         # band, S, R % G, g, r, 8
            .reshape(N, K))
    assert torch.equal(out.view(torch.int16), want.contiguous().view(torch.int16))


@pytest.mark.parametrize("mode", ["plain", "glu", "norm", "norm_glu", "residual"])
@pytest.mark.parametrize("M", [1, 17, 32, 64])
def test_swizzled_weight_same_bits(ie, dev, mode, M):
    """Every form of the skinny GEMM on the swizzled weight: bit for bit the row-major form's
    result at the same tile width (the gate/up forms, whose swizzled tiles pair 8 gate with 8 up
    rows, at half the width: the same output columns per workgroup; at odd widths, whose blocks
    the row-major form has no counterpart for, within the bound of another summation order)."""
    ops = ie.kernels.ops()
    glu = "glu" in mode
    N, K = (12288, 2048) if glu else (4096, 2048)
    h, gam, w = _norm_inputs(M, K, N, 500 + M, dev)
    for nt in ((1, 2, 3, 4) if glu else (1, 2, 4)):
        if nt + -(-M // 16) > 6:
            continue  # too wide for this many rows: refused for a swizzled weight
        sw = ie.swizzle_weight(w, nt, gate_up=glu)
        rm = max(1, nt // 2) if glu else nt  # the row-major width with the same blocks
        if mode == "plain":
            a, b = ops.skinny_matmul(h, w, nt, False), ops.skinny_matmul(h, sw, nt, True)
        elif mode == "glu":
            a = ops.skinny_matmul_silu_mul(h, w, rm, False)
            b = ops.skinny_matmul_silu_mul(h, sw, nt, True)
        elif mode in ("norm", "norm_glu"):
            a = ops.skinny_matmul_norm(h, w, rm, glu, EPS, False)
            b = ops.skinny_matmul_norm(h, sw, nt, glu, EPS, True)
        else:
            res0 = torch.randn(M, N, device=dev).bfloat16()
            a = ops.skinny_matmul_residual_(h, w, nt, res0.clone(), False)
            b = ops.skinny_matmul_residual_(h, sw, nt, res0.clone(), True)
        torch.cuda.synchronize()
        if glu and nt % 2:
            ref = a.float()
            bound = ref.abs() * 2 ** -7 + 2e-3 * ref.abs().max()
            assert torch.all((b.float() - ref).abs() <= bound), f"{mode} M={M} nt={nt}"
        else:
            assert torch.equal(a, b), f"{mode} M={M} nt={nt}"
    say(f"swizzled {mode} M={M}: ok")


@pytest.mark.parametrize("K", [2048, 1024])
@pytest.mark.parametrize("nt", [1, 2, 4])
def test_swizzled_wide_weight_looping_grid(ie, dev, nt, K):
    """A swizzled weight of many more row blocks than CUs (81,920 rows: 1,280 to 5,120 blocks,
    the LM head's case) runs on a grid of one looping workgroup per CU (at K = 2048 with each
    wave's x fragments held in registers over a fixed K slice): bit for bit the row-major
    one-block-per-workgroup result, at 32, 17 and 5 rows, plain and (K = 2048) with the RMSNorm
    inside."""
    ops = ie.kernels.ops()
    N = 81920
    g = torch.Generator().manual_seed(600 + nt + K)
    w = (0.02 * torch.randn(N, K, generator=g)).bfloat16().to(dev)
    sw = ie.swizzle_weight(w, nt)
    for M in (32, 17, 5):
        x = torch.randn(M, K, generator=g).bfloat16().to(dev)
        a, b = ops.skinny_matmul(x, w, nt, False), ops.skinny_matmul(x, sw, nt, True)
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"nt={nt} M={M}"
        # the RMSNorm form (the LM head with the final norm inside), likewise
        a = ops.skinny_matmul_norm(x, w, nt, False, EPS, False)
        b = ops.skinny_matmul_norm(x, sw, nt, False, EPS, True)
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"norm nt={nt} M={M}"


@pytest.mark.parametrize("M", [1, 17, 32, 64])
def test_fragment_order_activation(ie, dev, M):
    """The swizzled gate/up form's output in MFMA fragment order (IE_SKINNY_Y_FRAGMENTS) against
    the row-major output permuted on the CPU into the documented order (block S cdiv(M, 16) + t
    for column step S and row tile t, lane 16 g + r's 8 values: row 16 t + r, columns
    32 S + 8 g ..), bit for bit on the rows < M; and the down-projection-shaped residual GEMM
    reading it (IE_SKINNY_X_FRAGMENTS) equal to the same GEMM on the row-major activation, bit
    for bit, at every tile width, on the row-major and the swizzled weight."""
    ops = ie.kernels.ops()
    N, K = 12288, 2048
    h, gam, w = _norm_inputs(M, K, N, 700 + M, dev)
    mt = -(-M // 16)
    D = N // 2
    g = torch.Generator().manual_seed(701 + M)
    wd = (0.02 * torch.randn(2048, D, generator=g)).bfloat16().to(dev)
    res0 = torch.randn(M, 2048, generator=g).bfloat16().to(dev)
    for nt in (1, 2, 3, 4):
        if nt + mt > 6:
            continue
        sw = ie.swizzle_weight(w, nt, gate_up=True)
        rm = ops.skinny_matmul_norm(h, sw, nt, True, EPS, True)
        fr = ops.skinny_matmul_norm(h, sw, nt, True, EPS, True, True)
        torch.cuda.synchronize()
        assert fr.shape == (mt * 16, D)
        pad = torch.zeros(mt * 16, D, dtype=torch.bfloat16)
        pad[:M] = rm.cpu()
        want = pad.view(mt, 16, D // 32, 4, 8).permute(2, 0, 3, 1, 4).reshape(-1, 8)
        got = fr.cpu().reshape(-1, 8)
        rows = torch.arange(mt * 16).view(mt, 16)[None, :, None, :].expand(D // 32, mt, 4, 16)
        keep = (rows.reshape(-1) < M)  # rows past M are not written
        assert torch.equal(got[keep].view(torch.int16), want[keep].view(torch.int16)), \
            f"fragment order M={M} nt={nt}"
        for dnt in (0, 1, 2):
            for swz in ((False, True) if dnt else (False,)):
                wdd = ie.swizzle_weight(wd, dnt) if swz else wd
                if swz and dnt + mt > 6:
                    continue
                a = ops.skinny_matmul_residual_(rm, wdd, dnt, res0.clone(), swz)
                b = ops.skinny_matmul_residual_(fr, wdd, dnt, res0.clone(), swz, True)
                torch.cuda.synchronize()
                assert torch.equal(a, b), f"x fragments M={M} nt={nt} down nt={dnt} swz={swz}"
    say(f"fragment-order activation M={M}: bit-exact")


@pytest.mark.parametrize("M", [1, 17, 32])
def test_lm_head_greedy(ie, dev, M):
    """lm_head_greedy (the looping LM head with the greedy choice in the same launch): logits bit
    for bit those of linear_norm on the same reordered weight, tokens those of sample(logits, 0)
    on them, the seed advanced by one per call as sample advances it, at every tile width and
    on two calls in a row (the launch leaves its workspace zero). Planted: two equal columns
    that are every row's maximum, the later one in an earlier row block (the first column
    wins), and a NaN column (never chosen)."""
    K_ = ie.kernels
    N, K = 81920, 2048
    g = torch.Generator().manual_seed(900 + M)
    h = (torch.rand(M, K, generator=g) + 0.1).bfloat16().to(dev)  # positive rows
    w = (0.01 * torch.randn(N, K, generator=g))
    a, b, nan_col = 70000, 69840, 123
    w[a] = 0.05
    w[b] = 0.05
    w[nan_col] = float("nan")
    w = w.bfloat16().to(dev)
    for nt in (1, 2, 4):
        if nt + -(-M // 16) > 6:
            continue
        K_.use_skinny_swz[(N, K, M)] = nt
        sw = ie.swizzle_weight(w, nt)
        seed, seed_ref = (torch.full((1,), 5, dtype=torch.int64, device=dev) for _ in range(2))
        for call in range(2):
            logits, tok = ie.lm_head_greedy(h, sw, seed, EPS)
            ref = K_.linear_norm(h, sw, EPS, swizzled=True)
            want = ie.sample(ref, 0.0, seed_ref)
            torch.cuda.synchronize()
            assert torch.equal(logits.view(torch.int16), ref.view(torch.int16)), \
                f"logits M={M} nt={nt} call {call}"
            assert torch.equal(tok, want), f"tokens M={M} nt={nt} call {call}"
            assert torch.all(tok == b), f"tie: the first column wins, M={M} nt={nt}"
            assert seed.item() == seed_ref.item() == 6 + call
        K_.use_skinny_swz.pop((N, K, M))
    say(f"lm_head_greedy M={M}: bit-exact")
