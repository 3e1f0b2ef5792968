"""The attention layer of kbwal/inference-engine's Qwen3 model on this package's kernels: the
caller of every op in `kernels` (qwen3-1.7b/architecture.py:31-202), the RoPE tables it is fed
(architecture.py:343-354, 382-390), and the engine's graph capture of whole steps
(qwen3-1.7b/engine.py:105-117, 376-449).

`attention` is the body of AttentionLayer.forward between the QKV split and the output
projection, with the reference's dispatch (architecture.py:98):

  pure decode (cu_seqlens is None)   decode_attention_rope (= fused_rope_kv_decode ->
                                     decode_attention, one launch)
  step with prefill                  fused_norm_rope_prefill (every row) -> quantize_kv_prefill
                                     -> prefill_attention (prefix read from the int8 cache)
                                     -> decode_attention_rope(q[:B], out=out) with
                                        B = slot_ids.shape[0]: the decoding entries' rows of the
                                        prefill output (decoders come first, one token each, so
                                        decoding entry b is row b)

Two differences from the reference. The fused prefill kernel forces one: the
dequantize_kv_prefix call and its bf16 scratch (architecture.py:151-170) are gone, and
prefill_attention takes (kv_cache, slot_ids, cu_cached) instead; PrefixScratch keeps its fields
so the engine's call sites do not change, and only cu_cached is read. The other saves a launch
per layer: the reference's fused_rope_kv_decode and decode_attention calls run as one launch
that writes the same cache bits and attends with the same q bits.
"""

from dataclasses import dataclass
from typing import Callable

import torch
from torch.cuda import nvtx

from ._native import ops
from .kernels import (LayerKVCache, decode_attention_rope, fused_norm_rope_prefill, linear,
                      prefill_attention, quantize_kv_prefill)


@dataclass
class PrefixScratch:
    """qwen3-1.7b/architecture.py:19-27. k and v (the bf16 prefix copies) are not needed by the
    fused prefill kernel and may be None; cu_cached (int32 [S + 1]: entry b's prefix has
    cu_cached[b + 1] - cu_cached[b] tokens, 0 for decoders and unused entries) is read."""

    k: torch.Tensor | None
    v: torch.Tensor | None
    cu_cached: torch.Tensor


def rope_inv_freq(head_dim: int, base: float, device) -> torch.Tensor:
    """architecture.py:343-354: base^(-arange(0, D, 2) / D), fp32."""
    return base ** (-torch.arange(0, head_dim, 2, dtype=torch.float32, device=device) / head_dim)


def rope_tables(positions: torch.Tensor, inv_freq: torch.Tensor, dtype=torch.bfloat16):
    """architecture.py:382-390: angles = positions x inv_freq ([N, 1, D/2], fp32), then cos and
    sin cast to the activation dtype (bf16). A decode step's positions are its cached_lens.
    One launch (ie_rope_tables: the same fp32 product, cosf/sinf, round to nearest even)
    instead of PyTorch's five elementwise kernels."""
    assert dtype == torch.bfloat16
    if positions.dtype != torch.int32:
        positions = positions.int()
    return ops().rope_tables(positions, inv_freq)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, seq_ids, cu_seqlens,
              cos: torch.Tensor, sin: torch.Tensor, kv_cache: LayerKVCache,
              cached_lens: torch.Tensor, slot_ids: torch.Tensor, tile_start,
              prefill_block_m: int, prefix_scratch, num_decoding: torch.Tensor,
              q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor,
              eps: float = 1e-6, prefill_plan: torch.Tensor | None = None,
              decode_plan: torch.Tensor | None = None) -> torch.Tensor:
    """architecture.py:98-197. q [N, Hq, D], k/v [N, Hkv, D] (views of the QKV projection's
    output, before norm and RoPE). Returns [N, Hq, D]: in a step with prefill, rows of the
    prefilling entries from prefill attention and rows [0, num_decoding) from decode
    attention. prefill_plan: kernels.prefill_plan of the step's metadata, computed once per step
    for all layers (None: each prefill launch derives its work list itself); decode_plan:
    likewise kernels.decode_plan(cached_lens, num_decoding, len(slot_ids), Hq, Hkv) for the
    decode launch."""
    D = q.shape[-1]
    if cu_seqlens is None:
        # the reference's "rope_kv_write" and "decode_attention" ranges (architecture.py:100,
        # 115), one launch here
        with nvtx.range("rope_kv_write+decode_attention"):
            return decode_attention_rope(q, k, v, q_norm_weight, k_norm_weight, cos, sin,
                                         slot_ids, kv_cache, cached_lens, num_decoding, eps,
                                         D ** -0.5, plan=decode_plan)
    assert seq_ids is not None and tile_start is not None and prefix_scratch is not None
    # every kernel sees the whole packet and skips the entries that are not its own, so nothing
    # here depends on how many entries decode; the decode rows are normed and roped here too
    # (unused: the decode kernel below does its own)
    with nvtx.range("norm_rope_prefill"):
        q_p, k_p = fused_norm_rope_prefill(q, k, q_norm_weight, k_norm_weight, cos, sin, eps)
    with nvtx.range("kv_write"):
        quantize_kv_prefill(k_p, v, cu_seqlens, slot_ids, cached_lens, num_decoding, kv_cache)
    with nvtx.range("prefill_attention"):
        out = prefill_attention(q_p, k_p, v, seq_ids, cu_seqlens, tile_start, kv_cache,
                                slot_ids, prefix_scratch.cu_cached, prefill_block_m,
                                prefill_plan)
    B = slot_ids.shape[0]  # from a shape, not from how many entries decode
    with nvtx.range("rope_kv_write+decode_attention"):
        decode_attention_rope(q[:B], k[:B], v[:B], q_norm_weight, k_norm_weight, cos[:B],
                              sin[:B], slot_ids, kv_cache, cached_lens, num_decoding, eps,
                              D ** -0.5, out=out, plan=decode_plan)
    return out


class AttentionLayer:
    """qwen3-1.7b/architecture.py:31-202: QKV projection, `attention`, output projection.
    Weights: qkv [(Hq + 2 Hkv) D, model_dim], o_proj [model_dim, Hq D], q_norm/k_norm [D]
    (bf16); the projections go through `linear` (skinny GEMM or library GEMM, as tuned)."""

    def __init__(self, qkv: torch.Tensor, o_proj: torch.Tensor, q_norm: torch.Tensor,
                 k_norm: torch.Tensor, num_q_heads: int = 16, num_kv_heads: int = 8,
                 head_dim: int = 128, eps: float = 1e-6):
        self.qkv, self.o_proj, self.q_norm, self.k_norm = qkv, o_proj, q_norm, k_norm
        self.num_q_heads, self.num_kv_heads, self.head_dim, self.eps = (num_q_heads,
                                                                        num_kv_heads, head_dim,
                                                                        eps)

    def forward(self, x: torch.Tensor, seq_ids, cu_seqlens, cos, sin, kv_cache: LayerKVCache,
                cached_lens, slot_ids, tile_start, prefill_block_m: int, prefix_scratch,
                num_decoding) -> torch.Tensor:
        N = x.shape[0]
        D, hq, hkv = self.head_dim, self.num_q_heads, self.num_kv_heads
        with nvtx.range("qkv_proj"):
            q, k, v = linear(x, self.qkv).split([D * hq, D * hkv, D * hkv], dim=-1)
        out = attention(q.view(N, hq, D), k.view(N, hkv, D), v.view(N, hkv, D), seq_ids,
                        cu_seqlens, cos, sin, kv_cache, cached_lens, slot_ids, tile_start,
                        prefill_block_m, prefix_scratch, num_decoding, self.q_norm, self.k_norm,
                        self.eps)
        with nvtx.range("o_proj"):
            return linear(out.view(N, -1), self.o_proj)

    __call__ = forward


class GraphSet:
    """Whole-step hipGraphs in one memory pool (engine.py:105-117): the graphs reuse each other's
    intermediate memory, which is safe because only one replays at a time. `capture` warms the
    step up twice on a side stream, then records it (engine.py:432-449) and returns the graph
    and the output tensor every replay overwrites."""

    def __init__(self):
        self.pool = torch.cuda.graph_pool_handle()
        self.graphs: dict = {}
        # one side stream for every warm-up and capture: the ops' per-stream workspaces (zeroed
        # arrival counts) are then allocated by the first warm-up, outside any capture, and the
        # graphs share them as they share the pool (one replays at a time)
        self.stream = torch.cuda.Stream()

    def capture(self, key, run: Callable[[], torch.Tensor]):
        s = self.stream
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                run()
        torch.cuda.current_stream().wait_stream(s)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self.pool, stream=s):
            out = run()
        self.graphs[key] = (graph, out)
        return graph, out

    def replay(self, key) -> torch.Tensor:
        graph, out = self.graphs[key]
        graph.replay()
        return out
