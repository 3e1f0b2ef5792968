"""The attention kernel API of kbwal/inference-engine (qwen3-1.7b/kernels.py), on MI355X.

Same names, argument tensors, cache layout and host-side assertions as the reference's Python
wrappers; each call forwards to a torch.ops.ie op (lib/_ie_torch_ops.so), which forwards to the
C ABI of include/ie_attn.h (lib/libie_attn.so, hand-written gfx950 HIP). Nothing here computes on
the host, and there is no other code path: if the native libraries are missing the first call
raises.

Only one signature differs from the reference: `prefill_attention` reads each entry's cached
prefix straight from the int8 cache, so it takes (kv_cache, slot_ids, cu_cached) where the
reference took the bf16 prefix scratch (k_prefix, v_prefix, cu_cached) that
`dequantize_kv_prefix` filled (qwen3-1.7b/architecture.py:151-170). `dequantize_kv_prefix`
itself is still provided with the reference's signature.
"""

from dataclasses import dataclass

import torch

from ._native import ops


@dataclass
class LayerKVCache:
    """qwen3-1.7b/kernels.py:11-17."""

    k: torch.Tensor  # int8  [pool, Hkv, max_len, D]
    v: torch.Tensor  # int8  [pool, Hkv, max_len, D]
    k_scale: torch.Tensor  # fp32  [pool, Hkv, max_len]
    v_scale: torch.Tensor  # fp32  [pool, Hkv, max_len]
    k_calibration: torch.Tensor  # fp32  [pool, Hkv, 1, D]


def make_layer_cache(pool: int, num_kv_heads: int, max_len: int, head_dim: int,
                     device="cuda") -> LayerKVCache:
    """Zeroed cache with calibration ones (qwen3-1.7b/engine.py:472-492)."""
    return LayerKVCache(
        k=torch.zeros(pool, num_kv_heads, max_len, head_dim, device=device, dtype=torch.int8),
        v=torch.zeros(pool, num_kv_heads, max_len, head_dim, device=device, dtype=torch.int8),
        k_scale=torch.zeros(pool, num_kv_heads, max_len, device=device, dtype=torch.float32),
        v_scale=torch.zeros(pool, num_kv_heads, max_len, device=device, dtype=torch.float32),
        k_calibration=torch.ones(pool, num_kv_heads, 1, head_dim, device=device,
                                 dtype=torch.float32),
    )


def _cache_args(c: LayerKVCache):
    return c.k, c.v, c.k_scale, c.v_scale, c.k_calibration


def decode_attention(
    q: torch.Tensor,  # [B, Hq, D], one new token per sequence
    kv_cache: LayerKVCache,
    cached_lens: torch.Tensor,  # [B], tokens already cached per sequence
    slot_ids: torch.Tensor,  # [B], kv cache row of each sequence
    num_decoding: torch.Tensor,  # int32 [1], how many entries are decoding
    scale,
    out: torch.Tensor | None = None,  # [>= B, Hq, D]; decoding entry b's output goes to row b
    plan: torch.Tensor | None = None,  # decode_plan of this step's metadata (optional)
):
    """qwen3-1.7b/kernels.py:272-361. One launch on the current stream: the split-K kernel, whose
    last piece per sequence also does the reference's reduce (kernels.py:216-264). With `plan`
    (decode_plan over the same cached_lens / num_decoding values, batch and heads), each
    workgroup reads its work entry instead of deriving it: the same results."""
    k_cache, v_cache = kv_cache.k, kv_cache.v
    assert k_cache.stride() == v_cache.stride(), "kernel uses one set of strides for k and v"
    assert kv_cache.k_scale.stride() == kv_cache.v_scale.stride()
    B, Hq, D = q.shape
    if out is None:
        out = torch.empty(B, Hq, D, device=q.device, dtype=q.dtype)
    assert out.shape[0] >= B and out.shape[1:] == (Hq, D) and out.stride(-1) == 1
    ops().decode_attention(q, *_cache_args(kv_cache), cached_lens, slot_ids, num_decoding,
                           float(scale), out, plan)
    return out


def fused_rope_kv_decode(
    q: torch.Tensor,  # (B, Hq, D), one new token per sequence
    k: torch.Tensor,  # (B, Hkv, D)
    v: torch.Tensor,
    q_norm_weight: torch.Tensor,  # (D,)
    k_norm_weight: torch.Tensor,
    cos: torch.Tensor,  # (B, 1, D // 2)
    sin: torch.Tensor,
    slot_ids: torch.Tensor,  # [B]
    kv_cache: LayerKVCache,
    cached_lens: torch.Tensor,  # [B]
    num_decoding: torch.Tensor,
    eps: float,
):
    """qwen3-1.7b/kernels.py:483-544: returns normed + roped q (x calibration), writes K/V."""
    assert kv_cache.k.stride() == kv_cache.v.stride(), "kernel uses one set of strides for both caches"
    assert kv_cache.k_scale.stride() == kv_cache.v_scale.stride()
    return ops().fused_rope_kv_decode(q, k, v, q_norm_weight, k_norm_weight, cos, sin, slot_ids,
                                      *_cache_args(kv_cache), cached_lens, num_decoding,
                                      float(eps))


def decode_attention_rope(
    q: torch.Tensor,  # (B, Hq, D), the QKV projection's rows before norm and RoPE
    k: torch.Tensor,  # (B, Hkv, D)
    v: torch.Tensor,
    q_norm_weight: torch.Tensor,  # (D,)
    k_norm_weight: torch.Tensor,
    cos: torch.Tensor,  # (B, 1, D // 2)
    sin: torch.Tensor,
    slot_ids: torch.Tensor,  # [B]
    kv_cache: LayerKVCache,
    cached_lens: torch.Tensor,  # [B]
    num_decoding: torch.Tensor,
    eps: float,
    scale,
    out: torch.Tensor | None = None,  # [>= B, Hq, D]
    plan: torch.Tensor | None = None,  # decode_plan of this step's metadata (optional)
):
    """fused_rope_kv_decode (kernels.py:483-544) followed by decode_attention (kernels.py:272-361)
    in one launch: the same cache writes, bit for bit, and the attention of the q that
    fused_rope_kv_decode returns, which is not materialized. The decode branch of
    architecture.py:113-122 without the launch between the two ops. `plan` as for
    decode_attention."""
    assert kv_cache.k.stride() == kv_cache.v.stride(), "kernel uses one set of strides for both caches"
    assert kv_cache.k_scale.stride() == kv_cache.v_scale.stride()
    B, Hq, D = q.shape
    if out is None:
        out = torch.empty(B, Hq, D, device=q.device, dtype=q.dtype)
    assert out.shape[0] >= B and out.shape[1:] == (Hq, D) and out.stride(-1) == 1
    ops().decode_attention_rope(q, k, v, q_norm_weight, k_norm_weight, cos, sin,
                                *_cache_args(kv_cache), cached_lens, slot_ids, num_decoding,
                                float(eps), float(scale), out, plan)
    return out


def fused_norm_rope_prefill(
    q: torch.Tensor,  # bf16 [N, Hq, D], the prefill rows only: q[num_seqs_decoding:]
    k: torch.Tensor,  # bf16 [N, Hkv, D]
    q_norm_weight: torch.Tensor,  # [D]
    k_norm_weight: torch.Tensor,
    cos: torch.Tensor,  # [N, 1, D // 2]
    sin: torch.Tensor,
    eps: float,
) -> tuple:
    """qwen3-1.7b/kernels.py:665-714: normed + roped (q, k), contiguous."""
    assert q.stride(-1) == 1 and k.stride(-1) == 1, "kernel assumes contiguous head_dim"
    assert cos.stride(-1) == 1 and sin.stride(-1) == 1
    return ops().fused_norm_rope_prefill(q, k, q_norm_weight, k_norm_weight, cos, sin, float(eps))


def quantize_kv_prefill(
    k: torch.Tensor,  # bf16 [N, Hkv, D], all sequences packed along N
    v: torch.Tensor,  # bf16 [N, Hkv, D]
    cu_seqlens: torch.Tensor,  # int32 [B + 1]
    slot_ids: torch.Tensor,  # [B]
    cached_lens: torch.Tensor,  # [B]
    num_decoding: torch.Tensor,
    cache: LayerKVCache,
):
    """qwen3-1.7b/kernels.py:826-865."""
    N, Hkv, D = k.shape
    assert k.stride(-1) == 1 and v.stride(-1) == 1, "kernel assumes contiguous head_dim"
    assert cache.k.stride() == cache.v.stride()
    assert cache.k_scale.stride() == cache.v_scale.stride()
    ops().quantize_kv_prefill(k, v, cu_seqlens, slot_ids, cached_lens, num_decoding,
                              *_cache_args(cache))


def dequantize_kv_prefix(
    cache: LayerKVCache,
    cu_cached: torch.Tensor,  # int32 [B + 1]
    slot_ids: torch.Tensor,  # [B]
    k_out: torch.Tensor,  # bf16 [Hkv, >= total_cached, D]
    v_out: torch.Tensor,
):
    """qwen3-1.7b/kernels.py:935-970."""
    assert cache.k.stride() == cache.v.stride()
    assert cache.k_scale.stride() == cache.v_scale.stride()
    assert k_out.stride() == v_out.stride() and k_out.stride(-1) == 1
    ops().dequantize_kv_prefix(*_cache_args(cache), cu_cached, slot_ids, k_out, v_out)


def prefill_attention(
    q: torch.Tensor,  # bf16 [N, Hq, D], all sequences packed along N
    k: torch.Tensor,  # bf16 [N, Hkv, D]
    v: torch.Tensor,  # bf16 [N, Hkv, D]
    seq_ids: torch.Tensor,  # [N] which entry each packed token belongs to
    cu_seqlens: torch.Tensor,  # [B + 1] int32
    tile_start: torch.Tensor,  # [num_tiles] int32, first packed row of each tile
    kv_cache: LayerKVCache,  # entry b's prefix is cache row slot_ids[b]
    slot_ids: torch.Tensor,  # [B]
    cu_cached: torch.Tensor,  # [B + 1] int32, prefix lengths of every entry, cumulative
    PREFILL_BLOCK_M: int,  # must be the value tile_start was built with
    plan: torch.Tensor | None = None,  # prefill_plan(...) of the same metadata, or None
) -> torch.Tensor:
    """qwen3-1.7b/kernels.py:1129-1175 fused with the prefix dequantize (architecture.py:151-170).
    `plan` (not in the reference): the launch's work list from `prefill_plan` over the same
    step metadata and head counts; every workgroup then reads its item instead of deriving the
    list from the metadata. Same results."""
    N, Hq, D = q.shape
    assert q.stride(-1) == 1 and k.stride(-1) == 1 and v.stride(-1) == 1
    return ops().prefill_attention(q, k, v, seq_ids, cu_seqlens, tile_start,
                                   *_cache_args(kv_cache), slot_ids, cu_cached,
                                   int(PREFILL_BLOCK_M), plan)


def prefill_plan(seq_ids: torch.Tensor, cu_seqlens: torch.Tensor, tile_start: torch.Tensor,
                 slot_ids: torch.Tensor, cu_cached: torch.Tensor, num_tokens: int,
                 num_q_heads: int, num_kv_heads: int, PREFILL_BLOCK_M: int) -> torch.Tensor:
    """The work list of prefill_attention over one step's metadata ([grid, 16] int32 on the
    device, one row per workgroup: see ie_prefill_attention_plan), computed once per step and
    passed as `plan` to every layer's prefill_attention (no counterpart in the reference)."""
    return ops().prefill_plan(seq_ids, cu_seqlens, tile_start, slot_ids, cu_cached,
                              int(num_tokens), int(num_q_heads), int(num_kv_heads),
                              int(PREFILL_BLOCK_M))


def decode_plan(cached_lens: torch.Tensor, num_decoding: torch.Tensor, batch: int,
                num_q_heads: int, num_kv_heads: int) -> torch.Tensor:
    """The work list of decode_attention / decode_attention_rope over one step's metadata
    ([grid, 4] int32 on the device: see ie_decode_attention_plan), computed once per step and
    passed as `plan` to every layer's decode launch (no counterpart in the reference)."""
    return ops().decode_plan(cached_lens, num_decoding, int(batch), int(num_q_heads),
                             int(num_kv_heads))


def lm_head_greedy(h: torch.Tensor, weight: torch.Tensor, seed: torch.Tensor, eps: float = 0.0,
                   norm: bool = True):
    """The LM head and greedy sampling in one launch (ie_skinny_lm_head_greedy; no counterpart
    in the reference): (logits, tokens) with logits = linear_norm(h, weight, eps, swizzled=True)
    (norm; else skinny_matmul on the swizzled weight) and tokens = sample(logits, 0.0, seed)
    (which it also advances by one), the same bits as those calls. weight: swizzle_weight of the
    (norm-folded) LM head weight at swizzled_tiles' width; K = 2048, M <= 64."""
    M, K = h.shape
    N = weight.shape[0]
    nt = swizzled_tiles(N, K, M)
    assert nt in (1, 2, 4) and M <= 64 and K == 2048
    return ops().lm_head_greedy(h, weight, int(nt), float(eps), bool(norm), seed)


def decode_step_prologue(ids: torch.Tensor, embed: torch.Tensor, cached_lens: torch.Tensor,
                         num_decoding: torch.Tensor, num_q_heads: int, num_kv_heads: int,
                         inv_freq: torch.Tensor):
    """A decode step's per-step inputs in one launch (ie_decode_step_prologue; no counterpart
    in the reference): (x, plan, cos, sin) = (F.embedding(ids, embed), decode_plan(cached_lens,
    num_decoding, len(ids), num_q_heads, num_kv_heads), *rope_tables(cached_lens, inv_freq)),
    the same bits as those three calls."""
    return ops().decode_step_prologue(ids.reshape(-1), embed, cached_lens, num_decoding,
                                      int(num_q_heads), int(num_kv_heads), inv_freq)


def sample(logits: torch.Tensor, tau: float, seed: torch.Tensor) -> torch.Tensor:
    """qwen3-1.7b/kernels.py:1343-1370: [B, 1] int64 tokens (Gumbel-max; greedy at tau = 0);
    increments the int64 device `seed` by one."""
    B, V = logits.shape
    assert logits.stride(-1) == 1, "kernel assumes contiguous vocab dim"
    return ops().sample(logits, float(tau), seed)


def add_rms_norm(residual: torch.Tensor, delta: torch.Tensor, rms_norm: torch.Tensor, eps: float):
    """qwen3-1.7b/kernels.py:1260-1283: (bf16(residual + delta), its RMSNorm x weight)."""
    N, D = residual.shape
    assert residual.stride(-1) == 1 and delta.stride(-1) == 1
    return ops().add_rms_norm(residual, delta, rms_norm, float(eps))


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """qwen3-1.7b/kernels.py:1204-1213: [N, 2D] -> [N, D], silu(gate) * up."""
    return ops().silu_mul(gate_up)


def skinny_matmul(x: torch.Tensor, weight: torch.Tensor, n_tiles: int = 1,
                  swizzled: bool = False) -> torch.Tensor:
    """qwen3-1.7b/kernels.py:1406-1443: [M, K] bf16 @ [N, K].T bf16 -> [M, N] bf16 for M <= 64.
    `n_tiles` (1, 2, 4; 0 = 8 rows): weight rows per workgroup / 16, the launch shape tune_linear
    picks. swizzled: weight is swizzle_weight(W) (n_tiles 1, 2 or 4), the same result bits."""
    M, K = x.shape
    N = weight.shape[0]
    assert x.stride(-1) == 1 and weight.stride(-1) == 1
    assert M <= 64, "big M is compute bound, the library GEMM is faster there"
    assert n_tiles in (0, 1, 2, 4) and N % (16 * max(1, n_tiles)) == 0 and K % 256 == 0
    assert not swizzled or n_tiles >= 1
    return ops().skinny_matmul(x, weight, int(n_tiles), bool(swizzled))


def swizzle_weight(weight: torch.Tensor, n_tiles: int, gate_up: bool = False) -> torch.Tensor:
    """The weight in the skinny GEMM's fragment order for tile width n_tiles (1, 2 or 4;
    ie_skinny_weight_swizzle: 1 KB blocks of 16 rows x 32 columns that a wave loads whole,
    straight into MFMA operand registers, each workgroup's n_tiles row groups interleaved step by
    step). gate_up: the [gate; up] weight of the SiLU-gated form, its rows paired first (16-row
    tile R = gate rows 8R.. and the matching up rows; ie_skinny_weight_swizzle_gate_up; n_tiles
    1 ... 4, 8 n_tiles output columns per workgroup). Reordered once at load; the GEMMs then take
    it with swizzled=True and the same n_tiles (the tuned one, from the tables tune_linear
    fills). [N, K] like the weight (N a multiple of 16 n_tiles, K of 32), only for the skinny
    GEMM."""
    assert n_tiles in ((1, 2, 3, 4) if gate_up else (1, 2, 4))
    return ops().skinny_weight_swizzle(weight, int(n_tiles), bool(gate_up))


# (N, K, M) -> the n_tiles of skinny_matmul when it beat the library GEMM for that weight shape
# and row count, else None (qwen3-1.7b/kernels.py:1446-1448). Filled by tune_linear before graph
# capture; anything it never measured uses the library.
use_skinny: dict = {}
# (N, K, M) -> n_tiles of the fused gate/up + SiLU-gated launch, timed by tune_linear beside the
# plain choice (the fused launch's best tile width can differ from the plain GEMM's).
use_skinny_glu: dict = {}
# (N, K, M) -> n_tiles of the skinny GEMM on the weight reordered by swizzle_weight for that
# width, where tune_linear timed it faster than the row-major choice; None: keep the weight
# row-major. The _glu table holds the same for the fused gate/up launch on the weight reordered
# with gate_up=True (paired tiles of 8 output columns).
use_skinny_swz: dict = {}
use_skinny_glu_swz: dict = {}


def swizzled_tiles(N: int, K: int, M: int, silu_mul: bool = False):
    """The tile width to reorder an [N, K] weight for (swizzle_weight) and to run it with at M
    rows, or None where the row-major weight is the faster or nothing was tuned."""
    return (use_skinny_glu_swz if silu_mul else use_skinny_swz).get((N, K, M))


def skinny_matmul_silu_mul(x: torch.Tensor, weight: torch.Tensor, n_tiles: int = 1,
                           swizzled: bool = False) -> torch.Tensor:
    """silu_mul(skinny_matmul(x, weight)) in one launch (qwen3-1.7b/kernels.py:1451-1458 then
    :1178-1213): weight [2D, K] holds the gate rows then the up rows, result [M, D]."""
    M, K = x.shape
    N = weight.shape[0]
    assert x.stride(-1) == 1 and weight.stride(-1) == 1
    assert M <= 64 and N % 2 == 0
    if swizzled:  # swizzle_weight(..., gate_up=True): 8 n_tiles output columns per workgroup
        assert n_tiles in (1, 2, 3, 4) and (N // 2) % (8 * n_tiles) == 0 and K % 256 == 0
    else:
        assert n_tiles in (1, 2) and (N // 2) % (16 * n_tiles) == 0 and K % 256 == 0
    return ops().skinny_matmul_silu_mul(x, weight, int(n_tiles), bool(swizzled))


def linear_silu_mul(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """silu_mul(linear(x, weight)): the fused launch wherever tune_linear chose the skinny GEMM
    for this weight shape and row count, else the library GEMM then silu_mul."""
    key = (weight.shape[0], weight.shape[1], x.shape[0])
    if key in use_skinny_glu:
        return skinny_matmul_silu_mul(x, weight, use_skinny_glu[key])
    nt = use_skinny.get(key)
    if nt is not None and weight.shape[0] % 64 == 0:
        return skinny_matmul_silu_mul(x, weight, 2 if nt in (2, 4) else 1)
    return silu_mul(torch.nn.functional.linear(x, weight))


def fold_rms_norm_weight(weight: torch.Tensor, norm_weight: torch.Tensor) -> torch.Tensor:
    """bf16(W[n, k] * g[k]): the weight of a projection whose input is RMSNorm(h) * g, folded
    once (at load) for linear_norm, which then normalizes the rows inside the GEMM."""
    assert weight.dim() == 2 and norm_weight.shape == (weight.shape[1],)
    return (weight.float() * norm_weight.float()[None, :]).bfloat16()


def _skinny_tiles(table: dict, key: tuple, default: int) -> int:
    nt = table.get(key)
    return default if nt is None else nt


def linear_norm(h: torch.Tensor, weight_folded: torch.Tensor, eps: float,
                silu_mul: bool = False, swizzled: bool = False,
                fragments: bool = False) -> torch.Tensor:
    """linear(add_rms_norm's normed output, W) (silu_mul: then silu_mul, the gate/up form) from
    the residual stream h itself, in one skinny-GEMM launch (ie_skinny_gemm_fused with
    IE_SKINNY_NORM): weight_folded = fold_rms_norm_weight(W, g). The rows' sums of squares come
    from the GEMM's own reads of h, so the RMSNorm costs no launch (the reference runs
    add_rms_norm, kernels.py:1260-1283, before each such projection, architecture.py:280-300).
    M <= 64 rows; the tile width is the one tune_linear chose for the weight's shape (for a
    swizzled weight, swizzle_weight of the folded weight at swizzled_tiles' width, with gate_up
    for the SiLU-gated form). fragments (the swizzled SiLU-gated form): the output in MFMA
    fragment order ([cdiv(M, 16) 16, N / 2], IE_SKINNY_Y_FRAGMENTS), only for linear_residual_
    with x_fragments=True, which reads it without an LDS round trip."""
    M, K = h.shape
    N = weight_folded.shape[0]
    assert h.stride(-1) == 1 and weight_folded.stride(-1) == 1 and M <= 64
    key = (N, K, M)
    if silu_mul:
        nt = _skinny_tiles(use_skinny_glu, key, 1)
        if swizzled:  # paired tiles of 8 output columns: twice the row-major width
            nt = swizzled_tiles(N, K, M, True) or 2 * nt
            assert (N // 2) % (8 * nt) == 0 and K % 256 == 0
        else:
            assert (N // 2) % (16 * nt) == 0 and K % 256 == 0
    else:
        nt = _skinny_tiles(use_skinny, key, 1)
        if swizzled:
            nt = swizzled_tiles(N, K, M) or max(nt, 1)
        assert N % (16 * max(1, nt)) == 0 and K % 256 == 0
    assert not fragments or (silu_mul and swizzled)
    return ops().skinny_matmul_norm(h, weight_folded, int(nt), bool(silu_mul), float(eps),
                                    bool(swizzled), bool(fragments))


def linear_residual_(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor,
                     swizzled: bool = False, x_fragments: bool = False) -> torch.Tensor:
    """residual <- bf16(residual + linear(x, weight)) in place and returned: add_rms_norm's
    new residual for a projection's output (kernels.py:1240-1242), bit for bit, in the
    projection's own launch (ie_skinny_gemm_fused with IE_SKINNY_RESIDUAL). M <= 64 rows.
    x_fragments: x is linear_norm(..., fragments=True)'s output for the same rows (the same
    result bits)."""
    M, K = residual.shape[0], x.shape[1]
    N = weight.shape[0]
    assert x.stride(-1) == 1 and weight.stride(-1) == 1 and M <= 64
    assert residual.shape == (M, N) and residual.stride(-1) == 1
    nt = _skinny_tiles(use_skinny, (N, K, M), 1)
    if swizzled:
        nt = swizzled_tiles(N, K, M) or max(nt, 1)
    assert N % (16 * max(1, nt)) == 0 and K % 256 == 0
    return ops().skinny_matmul_residual_(x, weight, int(nt), residual, bool(swizzled),
                                         bool(x_fragments))


def linear(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """qwen3-1.7b/kernels.py:1451-1458: [M, K] @ [N, K].T -> [M, N], with whichever measured
    faster."""
    nt = use_skinny.get((weight.shape[0], weight.shape[1], x.shape[0]))
    if nt is not None:
        return skinny_matmul(x, weight, nt)
    return torch.nn.functional.linear(x, weight)


def tune_linear(weights: list, rows: list, calls: int = 20) -> None:
    """qwen3-1.7b/kernels.py:1461-1485: times skinny_matmul (each n_tiles) against the library
    GEMM for every weight shape at every row count and records the faster; the skinny kernel
    needs a 2 % win. Each candidate runs `calls` back-to-back launches captured in one hipGraph
    (the way the engine replays a step), cycling through copies of the weight that together
    exceed the 256 MB last-level cache, so the weights come from HBM as every layer's do in a
    step (the reference clears the cache before each timing for the same reason). Where the
    skinny kernel wins and N allows it, the fused gate/up + SiLU-gated launch is timed at each
    tile width as well, for linear_silu_mul; and both forms on the weight reordered by
    swizzle_weight at each width, recorded (use_skinny_swz, use_skinny_glu_swz) where faster than
    the row-major choice."""
    for weight in weights:
        N, K = weight.shape
        todo = [M for M in rows if M <= 64 and (N, K, M) not in use_skinny]
        if not todo:
            continue
        nbytes = weight.numel() * weight.element_size()
        copies = [weight] + [weight.clone() for _ in range(max(0, -(-(512 << 20) // nbytes) - 1))]
        for M in todo:
            x = torch.randn(M, K, device=weight.device, dtype=weight.dtype)
            cycle = lambda f, ws=copies: [lambda w=w: f(w) for w in ws] * max(1, calls // len(ws))
            lib = _graph_time(cycle(lambda w: torch.nn.functional.linear(x, w)))
            best, choice = 0.98 * lib, None
            if K % 256 == 0:
                for nt in (0, 1, 2, 4):
                    if N % (16 * max(1, nt)):
                        continue
                    t = _graph_time(cycle(lambda w, nt=nt: skinny_matmul(x, w, nt)))
                    if t < best:
                        best, choice = t, nt
            use_skinny[(N, K, M)] = choice
            glu = {}
            if choice is not None and N % 64 == 0:
                glu = {nt: _graph_time(cycle(lambda w, nt=nt: skinny_matmul_silu_mul(x, w, nt)))
                       for nt in (1, 2) if (N // 2) % (16 * nt) == 0}
                use_skinny_glu[(N, K, M)] = min(glu, key=glu.get)
            if choice is None:
                continue
            mt = -(-M // 16)  # the reordered weight's width cannot be lowered to fit the LDS
            swz, swz_glu = {}, {}
            for nt in (1, 2, 4):
                if N % (16 * nt) or nt + mt > 6:
                    continue
                sw = [swizzle_weight(w, nt) for w in copies]
                swz[nt] = _graph_time(cycle(lambda w, nt=nt: skinny_matmul(x, w, nt, True), sw))
                del sw
            for nt in ((1, 2, 3, 4) if glu else ()):  # paired gate/up tiles
                if (N // 2) % (8 * nt) or nt + mt > 6:
                    continue
                sw = [swizzle_weight(w, nt, gate_up=True) for w in copies]
                swz_glu[nt] = _graph_time(
                    cycle(lambda w, nt=nt: skinny_matmul_silu_mul(x, w, nt, True), sw))
                del sw
            pick = lambda t, ref: (min(t, key=t.get) if t and min(t.values()) < ref else None)
            use_skinny_swz[(N, K, M)] = pick(swz, best)
            if glu:
                use_skinny_glu_swz[(N, K, M)] = pick(swz_glu, min(glu.values()))
        del copies


def _graph_time(fns: list) -> float:
    """Average time per call of the calls `fns`, captured in order in one hipGraph."""
    for f in fns[:2]:
        f()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fns[0]()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        for f in fns:
            f()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(3):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (3 * len(fns))
